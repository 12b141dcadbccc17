"""The drop-in surface on the GPU: carl._carl.Env and CARLTorchVectorEnv.

Restates the reference's GPU tests (tests/test_gpu.py, test_gpu_backend.py,
test_stream_handoff.py and the ResetTests of test_resets.py) against this
engine: output shapes/dtypes/devices, truncation, stream ordering, the
combined reset against the individual setters, masked against indexed
resets, validation before mutation, the restored match clock, temporary
inputs on other streams, and the wrapper's terminal-successor and deferred
episode-report semantics.
"""
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

CURRENT = ("obs", "state", "score_difference", "episode_ticks", "overtime")
TRANSITION = ("transition_obs", "transition_state", "transition_score_difference", "transition_episode_ticks",
              "transition_overtime", "rewards", "dones")


def zeros(*shape, device="cuda"):
    return torch.zeros(shape, device=device, dtype=torch.float32)


def check_tensor(value, shape, dtype):
    assert isinstance(value, torch.Tensor) and value.is_cuda
    assert tuple(value.shape) == tuple(shape), (value.shape, shape)
    assert value.dtype == dtype
    assert torch.isfinite(value.float()).all().item()


def reset_inputs(n, n_cars, *, match=True, internal=True, device="cuda"):
    return fixtures.reset_inputs(n, n_cars, match=match, internal=internal, device=device)


def sequential_reset(env, values, indices):
    env.reset_boost_pads(indices)
    env.set_ball(values["ball_position"], values["ball_velocity"], values["ball_angular_velocity"],
                 simulation_indices=indices)
    env.set_car(values["car_position"], values["car_rotation"], values["car_velocity"],
                values["car_angular_velocity"], values["car_demoed"], boost=values.get("car_boost"),
                internal_state=values.get("car_internal_state"), simulation_indices=indices)
    if "blue_score" in values:
        env.set_match_state(values["blue_score"], values["orange_score"], values["episode_ticks"],
                            simulation_indices=indices)


def reset_provider(mask, *, typed, masked=False):
    indices = None if masked else mask.nonzero().flatten()
    count = len(mask) if masked else len(indices)
    values = reset_inputs(count, 2, device=mask.device)
    selection = {"reset_mask": mask} if masked else {"simulation_indices": indices}
    if not typed:
        return values | selection
    return typed_reset_state(values, indices, reset_mask=mask if masked else None)


def snapshot(env, names):
    torch.cuda.current_stream().wait_stream(torch.cuda.ExternalStream(env.stream))
    out = {name: torch.from_dlpack(getattr(env, "get_" + name)()).clone() for name in names}
    torch.cuda.synchronize()
    return out


def assert_same(actual, expected):
    torch.testing.assert_close(actual, expected, rtol=0, atol=0)


# ------------------------------------------------------------------ tests/test_gpu.py

def test_smoke_one_1v1_step(gpu):
    env = CARLTorchVectorEnv(n_sim=1, n_blue=1, n_orange=1, frameskip=1, discrete_actions=True, synchronize=True)
    try:
        observation = env.reset()
        assert isinstance(observation, CARLObservation)
        check_tensor(observation, env.observation_space.shape, torch.float32)
        check_tensor(observation.ball.position, (env.n_envs, 3), torch.float32)
        check_tensor(observation.cars.position, (env.n_envs, env.n_cars, 3), torch.float32)
        actions = torch.zeros((env.n_envs, len(carl.ACTION_NVECS)), dtype=torch.long, device=env.device)
        observation, reward, terminated, truncated, info = env.step(actions)
        assert isinstance(observation, CARLObservation)
        check_tensor(observation, env.observation_space.shape, torch.float32)
        check_tensor(reward, (env.n_envs,), torch.float32)
        check_tensor(terminated, (env.n_envs,), torch.bool)
        check_tensor(truncated, (env.n_envs,), torch.bool)
        assert isinstance(info, dict)
    finally:
        env.close()


# ------------------------------------------------------------------ tests/test_gpu_backend.py

@pytest.mark.parametrize("n_sim,discrete", [(17, False), (17, True), (8192, False)])
def test_outputs_and_truncation(gpu, n_sim, discrete):
    env = CARLTorchVectorEnv(n_sim=n_sim, n_blue=1, n_orange=1, discrete_actions=discrete, max_ticks=16,
                             overtime_timeout_ticks=8)
    dtype = torch.int64 if discrete else torch.float32
    actions = torch.zeros(env.action_space.shape, dtype=dtype, device=env.device)
    initial = env.reset()
    snapshot_initial = initial.clone()
    check_tensor(initial, env.observation_space.shape, torch.float32)
    assert torch.from_dlpack(env._env.get_obs()).__dlpack_device__() == (10, 0)
    saw_truncation = False
    for _ in range(8):
        obs, reward, terminated, truncated, _ = env.step(actions)
        check_tensor(obs, env.observation_space.shape, torch.float32)
        check_tensor(reward, (env.n_envs,), torch.float32)
        check_tensor(terminated, (env.n_envs,), torch.bool)
        check_tensor(truncated, (env.n_envs,), torch.bool)
        saw_truncation |= truncated.any().item()
    assert saw_truncation
    env.close()
    assert_same(initial, snapshot_initial)


# ------------------------------------------------------------------ tests/test_stream_handoff.py

def test_stream_handoff(gpu):
    def run(synchronize):
        env = CARLTorchVectorEnv(n_sim=4, n_blue=1, n_orange=1, seed=7, synchronize=synchronize)
        actions = torch.zeros(env.action_space.shape, device=env.device)
        frames = [env.reset().clone()]
        for step in range(8):
            if step == 4:
                z = torch.zeros((env.n_sim, 3), device=env.device)
                position = z.clone()
                position[:, 2] = 800.0
                env.set_ball(position, z, z)
                torch.cuda._sleep(50_000_000)
                frames.append(torch.from_dlpack(env._env.get_obs()).clone())
                obs = env.reset()
            else:
                obs = env.step(actions)[0]
            frames.append(obs.clone())
        env.close()
        return frames

    expected = run(synchronize=True)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        actual = run(synchronize=False)
    torch.cuda.synchronize()
    torch.testing.assert_close(actual, expected, rtol=1e-5, atol=1e-4)


# ------------------------------------------------------------------ tests/test_resets.py

@pytest.mark.parametrize("team_size,selection,optional", list(product((1, 2, 3), ([], [2, 0], None), (False, True))))
def test_combined_reset_matches_setters_and_continuation(gpu, team_size, selection, optional):
    reference = carl.Env(3, team_size, team_size, 7, previous_controls=True)
    env = carl.Env(3, team_size, team_size, 7, previous_controls=True)
    indices = None if selection is None else torch.tensor(selection, device="cuda", dtype=torch.int64)
    count = 3 if indices is None else len(indices)
    values = reset_inputs(count, 2 * team_size, match=optional, internal=optional)
    if not optional:
        values.pop("car_boost")
        values["car_demoed"] = values["car_demoed"].int()
    actions = zeros(3, 2 * team_size, 7)
    actions[..., 6] = 1  # held jump
    reference.no_touch_timeout_ticks = env.no_touch_timeout_ticks = 1
    reference.step_continuous(actions)
    env.step_continuous(actions)
    before = snapshot(env, CURRENT + TRANSITION)
    transition = {name: before[name] for name in TRANSITION}
    reference.no_touch_timeout_ticks = env.no_touch_timeout_ticks = 0
    for _ in range(2):
        sequential_reset(reference, values, indices)
        env.apply_reset_state(**values, simulation_indices=indices)
        assert_same(snapshot(env, TRANSITION), transition)
        assert_same(snapshot(env, ("obs", "state")), snapshot(reference, ("obs", "state")))
    after = snapshot(env, CURRENT)
    selected = range(3) if selection is None else selection
    untouched = sorted(set(range(3)) - set(selected))
    for name in CURRENT:
        assert_same(after[name][untouched], before[name][untouched])
    if optional and count:
        sel = slice(None) if indices is None else indices
        assert_same(after["score_difference"][sel], values["blue_score"] - values["orange_score"])
        assert_same(after["episode_ticks"][sel], values["episode_ticks"])
        assert not after["overtime"][sel].any().item()
    for _ in range(8):
        reference.step_continuous(actions)
        env.step_continuous(actions)
        assert_same(snapshot(env, CURRENT + TRANSITION), snapshot(reference, CURRENT + TRANSITION))


@pytest.mark.parametrize("masked", [False, True])
def test_contacts_use_complete_scene_without_physics(gpu, masked):
    env = carl.Env(1, 1, 1, 7, previous_controls=True)
    values = reset_inputs(1, 2)
    if masked:
        values["reset_mask"] = torch.ones(1, device="cuda", dtype=torch.bool)
    values["car_position"][0] = torch.tensor([[0, 0, 257], [0, 0, 200]], device="cuda")
    values["car_demoed"].zero_()
    env.apply_reset_state(**values)
    state = snapshot(env, ("state",))["state"]
    cars = state[:, carl.OBS_BALL:carl.OBS_BALL + 2 * carl.STATE_PER_CAR].view(1, 2, carl.STATE_PER_CAR)
    assert_same(cars[..., :3], values["car_position"])
    assert_same(cars[..., 3:6], values["car_velocity"])
    assert cars[0, 0, carl.OBS_ON_GROUND].item()
    assert not cars[0, 1, carl.OBS_ON_GROUND].item()
    assert not cars[..., carl.STATE_BALL_TOUCH].any().item()
    values["car_demoed"][:, 0] = True
    env.apply_reset_state(**values)
    obs = snapshot(env, ("obs",))["obs"]
    assert not obs[0, 0, carl.OBS_BALL + carl.OBS_ON_GROUND].item()


def test_rejects_invalid_input_before_mutation(gpu):
    env = carl.Env(2, 1, 1, 7)
    before = snapshot(env, CURRENT)
    values = reset_inputs(2, 2)
    bad_inputs = (
        {"episode_ticks": None},
        {"episode_ticks": values["episode_ticks"].long()},
        {"car_internal_state": torch.zeros((2, 2, 1), device="cuda")},
        {"car_position": values["car_position"].transpose(0, 1)},
        {"ball_velocity": torch.utils.dlpack.to_dlpack(values["ball_velocity"].cpu())},
        {"reset_mask": torch.ones(2, device="cuda")},
        {"reset_mask": torch.ones(3, device="cuda", dtype=torch.bool)},
        {"reset_mask": torch.ones(2, device="cuda", dtype=torch.bool), "simulation_indices": torch.arange(2, device="cuda")},
        {"reset_mask": torch.ones(2, device="cuda", dtype=torch.bool), "ball_position": values["ball_position"][:1]},
    )
    for bad in bad_inputs:
        with pytest.raises((ValueError, TypeError)):
            env.apply_reset_state(**(values | bad))
        assert_same(snapshot(env, CURRENT), before)


def test_restored_match_clock_enters_overtime_or_truncates(gpu):
    env = carl.Env(2, 1, 1, 7)
    env.max_ticks = 4
    env.overtime_timeout_ticks = 2
    values = reset_inputs(2, 2)
    values["orange_score"][0] = 2
    values["episode_ticks"].fill_(3)
    env.apply_reset_state(**values)
    actions = zeros(2, 2, 7)
    env.step_continuous(actions)
    out = snapshot(env, CURRENT + TRANSITION)
    assert_same(out["dones"], torch.tensor([False, True], device="cuda"))
    assert_same(out["overtime"], torch.tensor([True, False], device="cuda"))
    assert_same(out["transition_episode_ticks"], torch.tensor([4, 4], device="cuda", dtype=torch.int32))
    for _ in range(2):
        env.step_continuous(actions)
    out = snapshot(env, CURRENT + TRANSITION)
    assert_same(out["dones"], torch.tensor([True, False], device="cuda"))
    assert out["transition_overtime"][0].item()
    assert not out["overtime"].any().item()


def _reset_on_alternate_stream(*, capsules, masked=False):
    env = carl.Env(3, 1, 1, 7)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        values = reset_inputs(3 if masked else 2, 2)
        if masked:
            values["reset_mask"] = torch.tensor([True, False, True], device="cuda")
        else:
            values["simulation_indices"] = torch.tensor([2, 0], device="cuda")
        for i in range(4):
            torch.cuda._sleep(1_000_000)  # delay the producer: temporaries must survive native reads
            values["ball_position"][:, 0] = i * 100
            temporary = {name: value.clone() for name, value in values.items()}
            if capsules:
                torch.cuda.ExternalStream(env.stream).wait_stream(stream)
                temporary = {name: torch.utils.dlpack.to_dlpack(value) for name, value in temporary.items()}
            env.apply_reset_state(**temporary)
            del temporary
            scratch = [torch.empty_like(value).fill_(-999) for value in values.values()]
            del scratch
    torch.cuda.current_stream().wait_stream(stream)
    return snapshot(env, CURRENT)


def test_alternate_stream_temporary_inputs_and_capsules(gpu):
    expected = _reset_on_alternate_stream(capsules=False)
    for capsules, masked in product((False, True), repeat=2):
        got = _reset_on_alternate_stream(capsules=capsules, masked=masked)
        for name in CURRENT:
            assert_same(got[name], expected[name])


@pytest.mark.parametrize("team_size,mask", list(product((1, 2, 3), ([False, False, False], [True, False, True],
                                                                    [True, True, True]))))
def test_masked_reset_matches_indexed_reset(gpu, team_size, mask):
    reference = carl.Env(3, team_size, team_size, 7, previous_controls=True)
    env = carl.Env(3, team_size, team_size, 7, previous_controls=True)
    actions = zeros(3, 2 * team_size, 7)
    values = reset_inputs(3, 2 * team_size)
    mask = torch.tensor(mask, device="cuda")
    reference.no_touch_timeout_ticks = env.no_touch_timeout_ticks = 1
    reference.step_continuous(actions)
    env.step_continuous(actions)
    before = snapshot(env, TRANSITION)
    reference.no_touch_timeout_ticks = env.no_touch_timeout_ticks = 0
    for repeat in range(3):
        mask = mask.roll(1)
        indices = mask.nonzero().flatten()
        values["ball_position"][:, 0] = torch.arange(3, device="cuda") * 100 + repeat
        compact = {name: value[indices].contiguous() for name, value in values.items()}
        reference.apply_reset_state(**compact, simulation_indices=indices)
        env.apply_reset_state(**values, reset_mask=mask)
        assert_same(snapshot(env, CURRENT), snapshot(reference, CURRENT))
        assert_same(snapshot(env, TRANSITION), before)
    for _ in range(8):
        reference.step_continuous(actions)
        env.step_continuous(actions)
        assert_same(snapshot(env, CURRENT + TRANSITION), snapshot(reference, CURRENT + TRANSITION))


def test_close_waits_for_pending_masked_inputs(gpu):
    env = carl.Env(3, 1, 1, 7)
    stream = torch.cuda.ExternalStream(env.stream)
    complete = torch.cuda.Event()
    with torch.cuda.stream(stream):
        torch.cuda._sleep(1_000_000)
    env.apply_reset_state(**reset_inputs(3, 2), reset_mask=torch.ones(3, device="cuda", dtype=torch.bool))
    complete.record(stream)
    del env
    assert complete.query()


def _make_wrapper(**kwargs):
    return CARLTorchVectorEnv(n_sim=2, n_blue=1, n_orange=1, frameskip=1, no_touch_timeout_ticks=1, **kwargs)


@pytest.mark.parametrize("typed,goal,masked", list(product((False, True), repeat=3)))
def test_wrapper_preserves_terminal_successors(gpu, typed, goal, masked):
    control = _make_wrapper()
    candidate = _make_wrapper(masked_resets=masked)
    control.reset()
    candidate.reset()
    if goal:
        position = torch.tensor([[0, 5300, 100], [0, 5300, 100]], device="cuda", dtype=torch.float32)
        velocity = torch.zeros_like(position)
        control.set_ball(position, velocity, velocity)
        candidate.set_ball(position, velocity, velocity)
    provider = partial(reset_provider, typed=typed, masked=masked)
    candidate.reset_state_provider = provider
    actions = zeros(*control.action_space.shape)
    for completion in range(2):
        expected = control.step(actions)
        actual = candidate.step(actions)
        for a, e in zip(actual[1:4], expected[1:4]):
            assert_same(a, e)
        assert actual[4].keys() == expected[4].keys()
        for key in expected[4]:
            if isinstance(expected[4][key], torch.Tensor):
                assert_same(actual[4][key], expected[4][key])
            else:
                assert actual[4][key] == expected[4][key]
        done = actual[2] if (goal and completion == 0) else actual[3]
        assert done.all().item()
        t_cand, t_ctrl = snapshot(candidate._env, TRANSITION), snapshot(control._env, TRANSITION)
        for name in TRANSITION:
            assert_same(t_cand[name], t_ctrl[name])
        assert (actual[0].ball.position[:, 2] == 800).all().item()
        candidate.reset_state_provider = None
        candidate.reset()
        control.reset()
        candidate.reset_state_provider = provider
    candidate.close()
    control.close()


@pytest.mark.parametrize("copy_outputs", [False, True])
def test_deferred_episode_reports_match_immediate_reports(gpu, copy_outputs):
    reference = _make_wrapper(copy_outputs=copy_outputs)
    env = _make_wrapper(copy_outputs=copy_outputs, defer_episode_reporting=True)
    reference.reset()
    env.reset()
    actions = zeros(*env.action_space.shape)
    expected = {"reward": [], "length": []}
    for _ in range(5):
        control = reference.step(actions)
        with NoHostSync():
            actual = env.step(actions)
        for a, e in zip(actual[:4], control[:4]):
            assert_same(a, e)
        assert_same(actual[4]["final_obs"], control[4]["final_obs"])
        expected["reward"].extend(control[4]["reward"])
        expected["length"].extend(control[4]["length"])
        assert "reward" not in actual[4]
    assert env.drain_episode_reports() == expected
    assert len(expected["reward"]) == 5 * env.n_envs
    assert env.drain_episode_reports() == {"reward": [], "length": []}
    env.step(actions)
    env.reset()
    assert env.drain_episode_reports() == {"reward": [], "length": []}
    env.close()
    reference.close()
