"""Host-side Python layer on CPU tensors: state views and reset dispatch.

The behaviours of the reference's CPU checks (tests/test_state_views.py:8-38
and the ResetValidationTests of tests/test_resets.py:557-673), checked with
this suite's own structure and the reference's inputs and expected values:
  * ball, car and cars views read and write the observation tensor they were
    made from, at the observation layout's offsets, and the cars view exposes
    the per-car fields and the ego car;
  * with masked resets, CARLTorchVectorEnv hands the native environment the
    provider's fixed-shape inputs and the provider's mask ANDed with the
    eligible simulations, with no host readback and no compaction, for dict
    and typed providers alike, normalised typed inputs scaled back first;
  * a provider's selection metadata (mask dtype and length, a mask together
    with indices, indices on the masked path) is refused before anything
    reaches the native environment;
  * without masked resets, providers select rows by indices as before.
"""
from __future__ import annotations

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

# (view attribute, first column, end column) of the physics block every view shares
PHYSICS = (("position", carl.OBS_POS, carl.OBS_VEL), ("velocity", carl.OBS_VEL, carl.OBS_ANG),
           ("angular_velocity", carl.OBS_ANG, carl.OBS_FORWARD))


def _numbered(*shape):
    n = 1
    for s in shape:
        n *= s
    return torch.arange(n, dtype=torch.float32).reshape(shape)


def _raw_and_view(kind):
    if kind == "ball":
        raw = _numbered(2, carl.OBS_BALL)
        return raw, CARLBall.from_tensor(raw)
    if kind == "car":
        raw = _numbered(2, carl.OBS_PER_CAR)
        return raw, CARLCar.from_tensor(raw)
    raw = _numbered(2, 3, carl.OBS_PER_CAR)
    return raw, CARLCars.from_tensor(raw, 3)


@pytest.mark.parametrize("kind", ["ball", "car", "cars"])
def test_physics_views_alias_the_observation_columns(kind):
    raw, view = _raw_and_view(kind)
    for attr, lo, hi in PHYSICS:
        field = getattr(view, attr)
        assert torch.equal(field, raw[..., lo:hi]), attr
        # a write through the view lands in the observation tensor
        field.fill_(-1.0)
        assert bool((raw[..., lo:hi] == -1.0).all()), attr


def test_cars_view_exposes_car_fields_and_the_ego_car():
    raw = _numbered(2, 3, carl.OBS_PER_CAR)
    cars = CARLCars.from_tensor(raw, 3)
    assert cars.n_cars == 3
    expected = {
        "forward": raw[..., carl.OBS_FORWARD:carl.OBS_UP],
        "boost": raw[..., carl.OBS_BOOST],
        "on_ground": raw[..., carl.OBS_ON_GROUND].bool(),
    }
    for attr, want in expected.items():
        assert torch.equal(getattr(cars, attr), want), attr
    assert torch.equal(cars.ego.position, raw[:, 0, carl.OBS_POS:carl.OBS_VEL])


# ------------------------------------------------------------------ reset dispatch

def _bare_wrapper(provider, *, masked=True):
    """A CARLTorchVectorEnv of three 1v1 simulations whose native
    environment is a recording stand-in (nothing reaches a device)."""
    env = CARLTorchVectorEnv.__new__(CARLTorchVectorEnv)
    env.n_sim, env.n_cars = 3, 2
    env.masked_resets = masked
    env.reset_state_provider = provider
    env._env = mock.Mock()
    return env


def _native_call(env):
    env._env.apply_reset_state.assert_called_once()
    return env._env.apply_reset_state.call_args


ELIGIBLE = ((False, False, False), (True, False, True), (True, True, True))
PROVIDER_MASK = (True, True, False)


@pytest.mark.parametrize("typed,eligible", list(product((False, True), ELIGIBLE)))
def test_masked_dispatch_is_fixed_shape(typed, eligible):
    values = reset_inputs(3, 2)
    mask = torch.tensor(PROVIDER_MASK)
    answer = typed_reset_state(values, reset_mask=mask) if typed else {**values, "reset_mask": mask}
    provider = mock.Mock(return_value=answer)
    env = _bare_wrapper(provider)
    eligible = torch.tensor(eligible)
    with NoHostSync():
        env._apply_reset_state(eligible)
    provider.assert_called_once_with(eligible)
    args, kwargs = _native_call(env)
    # every simulation's row goes through, the mask picks the ones to reset
    assert kwargs["simulation_indices"] is None
    assert (tuple(args[0].shape), tuple(args[3].shape)) == ((3, 3), (3, 2, 3))
    torch.testing.assert_close(kwargs["reset_mask"], mask & eligible)
    torch.testing.assert_close(args[4], values["car_rotation"])


# provider answers whose selection the masked path must refuse
BAD_SELECTIONS = {
    "float mask": {"reset_mask": torch.ones(3)},
    "short mask": {"reset_mask": torch.ones(2, dtype=torch.bool)},
    "mask and indices": {"reset_mask": torch.ones(3, dtype=torch.bool), "simulation_indices": torch.arange(3)},
    "indices only": {"simulation_indices": torch.arange(3)},
}


@pytest.mark.parametrize("typed,bad", list(product((False, True), BAD_SELECTIONS)))
def test_masked_dispatch_refuses_bad_selections_first(typed, bad):
    values, selection = reset_inputs(3, 2), BAD_SELECTIONS[bad]
    if typed:
        answer = typed_reset_state(values, selection.get("simulation_indices"),
                                   reset_mask=selection.get("reset_mask"))
    else:
        answer = {**values, **selection}
    env = _bare_wrapper(mock.Mock(return_value=answer))
    with NoHostSync(), pytest.raises(ValueError):
        env._apply_reset_state(torch.ones(3, dtype=torch.bool))
    env._env.apply_reset_state.assert_not_called()


def test_normalised_typed_inputs_are_scaled_back_without_host_sync():
    values = reset_inputs(3, 2)
    mask = torch.tensor([True, False, True])
    answer = replace(typed_reset_state(values, reset_mask=mask), normalized=True)
    # the observation scales: positions by their per-axis scale, speeds by their maxima
    scale = torch.tensor(carl.OBS_POSITION_SCALE)
    for field, divisor in ((answer.ball.position, scale), (answer.ball.velocity, carl.BALL_MAX_SPEED),
                           (answer.ball.angular_velocity, carl.BALL_MAX_ANG_SPEED), (answer.cars.position, scale),
                           (answer.cars.velocity, carl.CAR_MAX_SPEED),
                           (answer.cars.angular_velocity, carl.CAR_MAX_ANG_SPEED),
                           (answer.cars.boost, carl.BOOST_MAX)):
        field.div_(divisor)
    env = _bare_wrapper(mock.Mock(return_value=answer))
    with NoHostSync():
        env._apply_reset_state(mask)
    args, kwargs = _native_call(env)
    for got, name in ((args[0], "ball_position"), (args[1], "ball_velocity"), (args[3], "car_position"),
                      (kwargs["car_boost"], "car_boost")):
        torch.testing.assert_close(got, values[name])


def _indexed_provider(mask, *, typed):
    rows = mask.nonzero().flatten()
    values = reset_inputs(len(rows), 2)
    return typed_reset_state(values, rows) if typed else {**values, "simulation_indices": rows}


@pytest.mark.parametrize("typed", [False, True])
def test_indexed_dispatch_selects_rows_by_index(typed):
    env = _bare_wrapper(partial(_indexed_provider, typed=typed), masked=False)
    env._apply_reset_state(torch.tensor([True, False, True]))
    args, kwargs = _native_call(env)
    assert tuple(args[0].shape) == (2, 3)
    assert kwargs["reset_mask"] is None
    torch.testing.assert_close(kwargs["simulation_indices"], torch.tensor([0, 2]))
