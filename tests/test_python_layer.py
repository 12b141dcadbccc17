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
from torch.utils._python_dispatch import TorchDispatchMode

import carl
from carl.gymnasium.state import CARLBall, CARLCar, CARLCars, CARLMatchReset, CARLResetState
from carl.gymnasium.torch import CARLTorchVectorEnv


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

def _zeros(*shape):
    return torch.zeros(shape, dtype=torch.float32)


def reset_inputs(n_selected, n_cars, *, match=True, internal=True):
    ball_position = _zeros(n_selected, 3)
    ball_position[:, 2] = 800
    ball_velocity = _zeros(n_selected, 3)
    ball_velocity[:, 0] = 170
    car_position = _zeros(n_selected, n_cars, 3)
    car_position[..., 0] = torch.arange(n_cars) * 250 - 500
    car_position[..., 1] = -1000
    car_position[..., 2] = 17
    car_rotation = _zeros(n_selected, n_cars, 4)
    car_rotation[..., 3] = 1
    demoed = torch.zeros((n_selected, n_cars), dtype=torch.bool)
    demoed[:, -1] = True
    out = {
        "ball_position": ball_position, "ball_velocity": ball_velocity,
        "ball_angular_velocity": _zeros(n_selected, 3), "car_position": car_position,
        "car_rotation": car_rotation, "car_velocity": _zeros(n_selected, n_cars, 3),
        "car_angular_velocity": _zeros(n_selected, n_cars, 3), "car_demoed": demoed,
        "car_boost": _zeros(n_selected, n_cars).fill_(61),
    }
    if internal:
        values = _zeros(n_selected, n_cars, carl.CAR_INTERNAL_SIZE)
        values[..., 3] = 1
        values[..., 5] = 1
        out["car_internal_state"] = values
    if match:
        out.update(blue_score=torch.full((n_selected,), 2, dtype=torch.int32),
                   orange_score=torch.full((n_selected,), 1, dtype=torch.int32),
                   episode_ticks=torch.full((n_selected,), 23, dtype=torch.int32))
    return out


def typed_reset_state(values, indices=None, *, reset_mask=None):
    ball = CARLBall.from_tensor(torch.cat((values["ball_position"], values["ball_velocity"],
                                           values["ball_angular_velocity"]), dim=-1))
    count, n_cars = values["car_position"].shape[:2]
    cars = CARLCars.from_tensor(_zeros(count, n_cars, carl.OBS_PER_CAR), n_cars)
    cars.position.copy_(values["car_position"])
    cars.forward[..., 0] = 1
    cars.up[..., 2] = 1
    cars.boost.copy_(values["car_boost"])
    cars[..., carl.OBS_DEMOED] = values["car_demoed"]
    match = CARLMatchReset(values["blue_score"], values["orange_score"], values["episode_ticks"])
    return CARLResetState(ball=ball, cars=cars, match=match, simulation_indices=indices, reset_mask=reset_mask,
                          car_internal_state=values.get("car_internal_state"))


def reset_provider(mask, *, typed):
    indices = mask.nonzero().flatten()
    values = reset_inputs(len(indices), 2)
    if not typed:
        return values | {"simulation_indices": indices}
    return typed_reset_state(values, indices)


class FixedShapeOnly(TorchDispatchMode):
    """Fail on scalar readback or dynamic compaction in the masked wrapper path."""

    def __torch_dispatch__(self, func, types, args=(), kwargs=None):
        forbidden = (torch.ops.aten._local_scalar_dense.default, torch.ops.aten.nonzero.default,
                     torch.ops.aten.masked_select.default, torch.ops.aten._unique2.default)
        if func in forbidden:
            raise AssertionError(f"host-dependent reset operation: {func}")
        if func == torch.ops.aten.index.Tensor:
            if any(i is not None and i.dtype in (torch.bool, torch.uint8) for i in args[1]):
                raise AssertionError("boolean reset compaction")
        return func(*args, **(kwargs or {}))


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
    with FixedShapeOnly():
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
    with FixedShapeOnly(), pytest.raises(ValueError):
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
    with FixedShapeOnly():
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
