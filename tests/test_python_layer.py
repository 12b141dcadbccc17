"""Host-side Python layer on CPU tensors: state views and reset dispatch.

Mirrors the reference's CPU checks (tests/test_state_views.py and the
ResetValidationTests of tests/test_resets.py): views share storage and keep
the observation layout, and the masked reset path of CARLTorchVectorEnv stays
fixed-shape (no host readback, no compaction) and validates its metadata
before anything reaches the native environment.
"""
from dataclasses import replace
from functools import partial
from itertools import product
from unittest import mock

import pytest
import torch

import carl
from carl.gymnasium.state import CARLBall, CARLCar, CARLCars
from carl.gymnasium.torch import CARLTorchVectorEnv
from reset_fixtures import NoHostSync, reset_inputs, typed_reset_state


# ------------------------------------------------------------------ state views

def _assert_view(raw, view, start, end):
    assert torch.equal(view, raw[..., start:end])
    view.fill_(-1)
    assert (raw[..., start:end] == -1).all()


def test_physics_views_share_storage_and_preserve_layout():
    ball = torch.arange(2 * carl.OBS_BALL, dtype=torch.float32).reshape(2, carl.OBS_BALL)
    car = torch.arange(2 * carl.OBS_PER_CAR, dtype=torch.float32).reshape(2, carl.OBS_PER_CAR)
    cars = torch.arange(6 * carl.OBS_PER_CAR, dtype=torch.float32).reshape(2, 3, carl.OBS_PER_CAR)
    for raw, state in ((ball, CARLBall.from_tensor(ball)), (car, CARLCar.from_tensor(car)),
                       (cars, CARLCars.from_tensor(cars, 3))):
        _assert_view(raw, state.position, carl.OBS_POS, carl.OBS_VEL)
        _assert_view(raw, state.velocity, carl.OBS_VEL, carl.OBS_ANG)
        _assert_view(raw, state.angular_velocity, carl.OBS_ANG, carl.OBS_FORWARD)


def test_cars_inherit_car_fields_and_ego():
    raw = torch.arange(2 * 3 * carl.OBS_PER_CAR, dtype=torch.float32).reshape(2, 3, carl.OBS_PER_CAR)
    cars = CARLCars.from_tensor(raw, 3)
    assert cars.n_cars == 3
    assert torch.equal(cars.forward, raw[..., carl.OBS_FORWARD:carl.OBS_UP])
    assert torch.equal(cars.boost, raw[..., carl.OBS_BOOST])
    assert torch.equal(cars.ego.position, raw[:, 0, carl.OBS_POS:carl.OBS_VEL])
    assert torch.equal(cars.on_ground, raw[..., carl.OBS_ON_GROUND].bool())


# ------------------------------------------------------------------ reset dispatch

def reset_provider(mask, *, typed):
    indices = mask.nonzero().flatten()
    values = reset_inputs(len(indices), 2)
    if not typed:
        return values | {"simulation_indices": indices}
    return typed_reset_state(values, indices)


def make_env(provider, masked=True):
    env = CARLTorchVectorEnv.__new__(CARLTorchVectorEnv)
    env.n_sim = 3
    env.n_cars = 2
    env.masked_resets = masked
    env.reset_state_provider = provider
    env._env = mock.Mock()
    return env


@pytest.mark.parametrize("typed,eligible", list(product((False, True), ([False, False, False], [True, False, True],
                                                                          [True, True, True]))))
def test_masked_provider_never_compacts_or_reads_scalars(typed, eligible):
    values = reset_inputs(3, 2)
    mask = torch.tensor([True, True, False])
    eligible = torch.tensor(eligible)
    state = typed_reset_state(values, reset_mask=mask) if typed else values | {"reset_mask": mask}
    provider = mock.Mock(return_value=state)
    env = make_env(provider)
    with NoHostSync():
        env._apply_reset_state(eligible)
    provider.assert_called_once_with(eligible)
    env._env.apply_reset_state.assert_called_once()
    args, kwargs = env._env.apply_reset_state.call_args
    assert kwargs["simulation_indices"] is None
    assert args[0].shape == (3, 3)
    assert args[3].shape == (3, 2, 3)
    torch.testing.assert_close(kwargs["reset_mask"], mask & eligible)
    torch.testing.assert_close(args[4], values["car_rotation"])


INVALID = ({"reset_mask": torch.ones(3)}, {"reset_mask": torch.ones(2, dtype=torch.bool)},
           {"reset_mask": torch.ones(3, dtype=torch.bool), "simulation_indices": torch.arange(3)},
           {"simulation_indices": torch.arange(3)})


@pytest.mark.parametrize("typed,selection", list(product((False, True), INVALID)))
def test_masked_provider_validates_selection_metadata(typed, selection):
    values = reset_inputs(3, 2)
    if typed:
        state = typed_reset_state(values, selection.get("simulation_indices"),
                                  reset_mask=selection.get("reset_mask"))
    else:
        state = values | selection
    env = make_env(mock.Mock(return_value=state))
    with NoHostSync(), pytest.raises(ValueError):
        env._apply_reset_state(torch.ones(3, dtype=torch.bool))
    env._env.apply_reset_state.assert_not_called()


def test_normalized_masked_inputs_remain_fixed_shape():
    values = reset_inputs(3, 2)
    mask = torch.tensor([True, False, True])
    state = replace(typed_reset_state(values, reset_mask=mask), normalized=True)
    scale = torch.tensor(carl.OBS_POSITION_SCALE)
    state.ball.position.div_(scale)
    state.ball.velocity.div_(carl.BALL_MAX_SPEED)
    state.ball.angular_velocity.div_(carl.BALL_MAX_ANG_SPEED)
    state.cars.position.div_(scale)
    state.cars.velocity.div_(carl.CAR_MAX_SPEED)
    state.cars.angular_velocity.div_(carl.CAR_MAX_ANG_SPEED)
    state.cars.boost.div_(carl.BOOST_MAX)
    env = make_env(mock.Mock(return_value=state))
    with NoHostSync():
        env._apply_reset_state(mask)
    args, kwargs = env._env.apply_reset_state.call_args
    torch.testing.assert_close(args[0], values["ball_position"])
    torch.testing.assert_close(args[1], values["ball_velocity"])
    torch.testing.assert_close(args[3], values["car_position"])
    torch.testing.assert_close(kwargs["car_boost"], values["car_boost"])


@pytest.mark.parametrize("typed", [False, True])
def test_indexed_providers_remain_supported(typed):
    env = make_env(partial(reset_provider, typed=typed), masked=False)
    env._apply_reset_state(torch.tensor([True, False, True]))
    args, kwargs = env._env.apply_reset_state.call_args
    assert args[0].shape == (2, 3)
    assert kwargs["reset_mask"] is None
    torch.testing.assert_close(kwargs["simulation_indices"], torch.tensor([0, 2]))
