"""Named tensor views over CARL's packed observation and state layouts.

API-compatible with the reference views (python/carl/gymnasium/state.py:10-530):
the same classes and properties, each a slice that shares storage with the
packed tensor.  Offsets come from the module constants, which restate the
layout contract of include/Cuda/DLPack.h:60-107.
"""
from __future__ import annotations

from collections.abc import Mapping
from dataclasses import dataclass, field
from typing import Any

import torch as th

import carl_amd as carl
from carl_amd import BOOST_PAD_POSITIONS, REGULATION_TICKS


@dataclass(frozen=True)
class RewardResult:
    reward: th.Tensor
    info: Mapping[str, list[Any]] = field(default_factory=dict)


class _CARLTensor(th.Tensor):
    """Tensor subclass whose torch operations return plain tensors."""

    @classmethod
    def from_tensor(cls, tensor: th.Tensor):
        return tensor.as_subclass(cls)

    @classmethod
    def __torch_function__(cls, func, types, args=(), kwargs=None):
        with th._C.DisableTorchFunctionSubclass():
            return func(*args, **(kwargs or {}))


def _span(start: int, stop: int, doc: str):
    return property(lambda self: self[..., start:stop], doc=doc)


def _scalar(index: int, doc: str, as_bool: bool = False):
    if as_bool:
        return property(lambda self: self[..., index].bool(), doc=doc)
    return property(lambda self: self[..., index], doc=doc)


class _CARLPhysics(_CARLTensor):
    position = _span(carl.OBS_POS, carl.OBS_VEL, "position (uu)")
    velocity = _span(carl.OBS_VEL, carl.OBS_ANG, "linear velocity (uu/s)")
    angular_velocity = _span(carl.OBS_ANG, carl.OBS_FORWARD, "angular velocity (rad/s)")


class CARLBall(_CARLPhysics):
    pass


class CARLCar(_CARLPhysics):
    forward = _span(carl.OBS_FORWARD, carl.OBS_UP, "forward axis")
    up = _span(carl.OBS_UP, carl.OBS_BOOST, "up axis")
    boost = _scalar(carl.OBS_BOOST, "boost amount")
    on_ground = _scalar(carl.OBS_ON_GROUND, "three or more wheels in contact", True)
    demoed = _scalar(carl.OBS_DEMOED, "demolished", True)
    has_flipped = _scalar(carl.OBS_HAS_FLIPPED, "flip used", True)
    has_double_jumped = _scalar(carl.OBS_HAS_DOUBLE_JUMPED, "double jump used", True)
    is_boosting = _scalar(carl.OBS_IS_BOOSTING, "boosting", True)


class CARLCars(CARLCar):
    """[..., n_cars, OBS_PER_CAR] view; car 0 is the observer."""

    @staticmethod
    def from_tensor(tensor: th.Tensor, n_cars: int) -> "CARLCars":
        cars = tensor.as_subclass(CARLCars)
        cars._n_cars = n_cars
        return cars

    @property
    def n_cars(self) -> int:
        return self._n_cars

    @property
    def ego(self) -> CARLCar:
        return CARLCar.from_tensor(self[..., 0, :])

    ego_position = property(lambda self: self.ego.position)
    ego_velocity = property(lambda self: self.ego.velocity)
    ego_angular_velocity = property(lambda self: self.ego.angular_velocity)
    ego_forward = property(lambda self: self.ego.forward)
    ego_up = property(lambda self: self.ego.up)
    ego_boost = property(lambda self: self.ego.boost)


class CARLObservation(_CARLTensor):
    """One agent's packed observation with named views."""

    _n_cars: int

    @staticmethod
    def from_tensor(tensor: th.Tensor, n_cars: int) -> "CARLObservation":
        obs = tensor.as_subclass(CARLObservation)
        obs._n_cars = n_cars
        return obs

    @property
    def n_cars(self) -> int:
        return self._n_cars

    @property
    def car_end(self) -> int:
        return carl.OBS_BALL + carl.OBS_PER_CAR * self._n_cars

    # ball
    @property
    def ball(self) -> CARLBall:
        return CARLBall.from_tensor(self[..., :carl.OBS_BALL])

    ball_values = property(lambda self: self.ball)
    ball_position = property(lambda self: self.ball.position)
    ball_velocity = property(lambda self: self.ball.velocity)
    ball_angular_velocity = property(lambda self: self.ball.angular_velocity)

    # cars: observer, teammates, opponents
    @property
    def cars(self) -> CARLCars:
        flat = self[..., carl.OBS_BALL:self.car_end]
        return CARLCars.from_tensor(flat.view(*self.shape[:-1], self._n_cars, carl.OBS_PER_CAR), self._n_cars)

    car_values = property(lambda self: self.cars)
    ego_values = property(lambda self: self.cars.ego)
    car_position = property(lambda self: self.cars.position)
    car_velocity = property(lambda self: self.cars.velocity)
    car_angular_velocity = property(lambda self: self.cars.angular_velocity)
    car_forward = property(lambda self: self.cars.forward)
    car_up = property(lambda self: self.cars.up)
    car_boost = property(lambda self: self.cars.boost)
    car_on_ground = property(lambda self: self.cars.on_ground)
    car_demoed = property(lambda self: self.cars.demoed)
    car_has_flipped = property(lambda self: self.cars.has_flipped)
    car_has_double_jumped = property(lambda self: self.cars.has_double_jumped)
    car_is_boosting = property(lambda self: self.cars.is_boosting)

    # boost pads
    @property
    def boost_pad_active(self) -> th.Tensor:
        return self[..., self.car_end:self.car_end + carl.NUM_BOOST_PADS].bool()

    @property
    def boost_pad_distance(self) -> th.Tensor:
        start = self.car_end + carl.NUM_BOOST_PADS
        return self[..., start:start + carl.NUM_BOOST_PADS]

    # relative vectors
    @property
    def ego_ball_relative(self) -> th.Tensor:
        start = self.car_end + carl.OBS_BOOST_PADS
        return self[..., start:start + carl.OBS_RELATIVE_EGO_BALL]

    @property
    def ego_other_relative(self) -> th.Tensor:
        start = self.car_end + carl.OBS_BOOST_PADS + carl.OBS_RELATIVE_EGO_BALL
        stop = start + carl.OBS_RELATIVE_PER_OTHER_CAR * (self._n_cars - 1)
        return self[..., start:stop].view(*self.shape[:-1], self._n_cars - 1, carl.OBS_RELATIVE_PER_OTHER_CAR)

    @property
    def _goal_start(self) -> int:
        return (self.car_end + carl.OBS_BOOST_PADS + carl.OBS_RELATIVE_EGO_BALL
                + carl.OBS_RELATIVE_PER_OTHER_CAR * (self._n_cars - 1))

    @property
    def own_goal_relative(self) -> th.Tensor:
        return self[..., self._goal_start:self._goal_start + carl.OBS_VECTOR_SIZE]

    @property
    def opponent_goal_relative(self) -> th.Tensor:
        start = self._goal_start + carl.OBS_VECTOR_SIZE
        return self[..., start:start + carl.OBS_VECTOR_SIZE]

    # dodge window and controller state
    @property
    def ego_has_flip_or_jump(self) -> th.Tensor:
        return self[..., self._goal_start + carl.OBS_RELATIVE_GOALS].bool()

    @property
    def ego_flip_window_remaining(self) -> th.Tensor:
        return self[..., self._goal_start + carl.OBS_RELATIVE_GOALS + 1]

    @property
    def ego_controller(self) -> th.Tensor:
        start = self._goal_start + carl.OBS_RELATIVE_GOALS + carl.OBS_EGO_DODGE
        stop = start + carl.OBS_EGO_CONTROLLER
        if self.shape[-1] not in (stop, stop + carl.OBS_PREVIOUS_CONTROLS):
            raise ValueError("observation does not match ego controller v3")
        return self[..., start:stop]

    @property
    def ego_previous_controls(self) -> th.Tensor:
        self.ego_controller  # validates the layout
        start = self._goal_start + carl.OBS_RELATIVE_GOALS + carl.OBS_EGO_DODGE + carl.OBS_EGO_CONTROLLER
        if self.shape[-1] != start + carl.OBS_PREVIOUS_CONTROLS:
            raise ValueError("observation does not include previous controls")
        return self[..., start:]

    ego_has_jumped = property(lambda self: self.ego_controller[..., 0].bool())
    ego_is_jumping = property(lambda self: self.ego_controller[..., 1].bool())
    ego_is_flipping = property(lambda self: self.ego_controller[..., 2].bool())
    ego_flip_time = property(lambda self: self.ego_controller[..., 3])
    ego_demo_respawn_time = property(lambda self: self.ego_controller[..., 4])


@dataclass(frozen=True)
class CARLMatchReset:
    """Match state of the simulations a reset provider restores."""

    blue_score: th.Tensor
    orange_score: th.Tensor
    episode_ticks: th.Tensor


@dataclass(frozen=True)
class CARLResetState:
    """Reset state in physics units (or normalised units when ``normalized``).

    Indexed form: ``simulation_indices`` (int64) names the rows.  Fixed-shape
    form: ``simulation_indices=None`` and a bool ``reset_mask`` [n_sim]; every
    tensor then has one row per arena and only metadata is validated on the
    host.
    """

    simulation_indices: th.Tensor | None
    ball: CARLBall
    cars: CARLCars
    car_internal_state: th.Tensor | None = None
    match: CARLMatchReset | None = None
    normalized: bool = False
    reset_mask: th.Tensor | None = None

    def validate(self, reset_mask: th.Tensor, n_cars: int) -> None:
        rows = len(reset_mask)
        if self.reset_mask is not None:
            if self.simulation_indices is not None:
                raise ValueError("specify reset_mask or simulation_indices, not both")
            mask = self.reset_mask
            if mask.shape != reset_mask.shape or mask.dtype != th.bool or mask.device != reset_mask.device:
                raise ValueError("reset_mask must be bool [n_sim] on the environment device")
        else:
            self._validate_indices(reset_mask)
            rows = len(self.simulation_indices)
        if self.ball.shape != (rows, carl.OBS_BALL) or self.cars.shape != (rows, n_cars, carl.OBS_PER_CAR):
            raise ValueError("ball or cars have the wrong shape")

    def _validate_indices(self, reset_mask: th.Tensor) -> None:
        idx = self.simulation_indices
        if idx is None or idx.ndim != 1 or idx.dtype != th.int64 or idx.device != reset_mask.device:
            raise ValueError("simulation_indices must be int64 on the environment device")
        if ((idx < 0) | (idx >= len(reset_mask))).any():
            raise ValueError("simulation_indices are out of range")
        if not reset_mask[idx].all() or th.unique(idx).numel() != len(idx):
            raise ValueError("simulation_indices must be unique and selected for reset")

    def physical(self) -> tuple[CARLBall, CARLCars]:
        if not self.normalized:
            return self.ball, self.cars
        ball = CARLBall.from_tensor(self.ball.clone())
        cars = CARLCars.from_tensor(self.cars.clone(), self.cars.n_cars)
        scale = ball.position.new_tensor(carl.OBS_POSITION_SCALE)
        ball.position.mul_(scale)
        ball.velocity.mul_(carl.BALL_MAX_SPEED)
        ball.angular_velocity.mul_(carl.BALL_MAX_ANG_SPEED)
        cars.position.mul_(scale)
        cars.velocity.mul_(carl.CAR_MAX_SPEED)
        cars.angular_velocity.mul_(carl.CAR_MAX_ANG_SPEED)
        cars.boost.mul_(carl.BOOST_MAX)
        return ball, cars


def _state_span(start: int, stop: int):
    return property(lambda self: self.car_values[..., start:stop])


def _state_flag(index: int, as_bool: bool = True):
    if as_bool:
        return property(lambda self: self.car_values[..., index].bool())
    return property(lambda self: self.car_values[..., index])


@dataclass(frozen=True)
class CarlState:
    """Canonical (un-mirrored) per-simulation state, [n_sim, state_dim]."""

    raw: th.Tensor
    n_cars: int
    boost_pad_positions: th.Tensor
    team_sign: th.Tensor

    @classmethod
    def from_raw(cls, raw: th.Tensor, n_cars: int, boost_pad_positions: th.Tensor,
                 team_sign: th.Tensor) -> "CarlState":
        expected = carl.OBS_BALL + carl.STATE_PER_CAR * n_cars + carl.NUM_BOOST_PADS
        if raw.ndim != 2 or raw.shape[1] != expected:
            raise ValueError(f"Expected raw state shaped [n_sim, {expected}], got {tuple(raw.shape)}")
        return cls(raw, n_cars, boost_pad_positions, team_sign)

    @property
    def ball_values(self) -> th.Tensor:
        return self.raw[:, :carl.OBS_BALL]

    ball_position = property(lambda self: self.ball_values[..., carl.OBS_POS:carl.OBS_VEL])
    ball_velocity = property(lambda self: self.ball_values[..., carl.OBS_VEL:carl.OBS_ANG])
    ball_angular_velocity = property(lambda self: self.ball_values[..., carl.OBS_ANG:carl.OBS_BALL])

    @property
    def car_values(self) -> th.Tensor:
        stop = carl.OBS_BALL + carl.STATE_PER_CAR * self.n_cars
        return self.raw[:, carl.OBS_BALL:stop].view(self.raw.shape[0], self.n_cars, carl.STATE_PER_CAR)

    car_position = _state_span(carl.OBS_POS, carl.OBS_VEL)
    car_velocity = _state_span(carl.OBS_VEL, carl.OBS_ANG)
    car_angular_velocity = _state_span(carl.OBS_ANG, carl.OBS_FORWARD)
    car_forward = _state_span(carl.OBS_FORWARD, carl.OBS_UP)
    car_up = _state_span(carl.OBS_UP, carl.OBS_BOOST)
    car_boost = _state_flag(carl.OBS_BOOST, as_bool=False)
    car_on_ground = _state_flag(carl.OBS_ON_GROUND)
    car_demoed = _state_flag(carl.OBS_DEMOED)
    car_has_flipped = _state_flag(carl.OBS_HAS_FLIPPED)
    car_has_double_jumped = _state_flag(carl.OBS_HAS_DOUBLE_JUMPED)
    car_is_boosting = _state_flag(carl.OBS_IS_BOOSTING)
    car_ball_touches = _state_flag(carl.STATE_BALL_TOUCH)

    @property
    def boost_pad_values(self) -> th.Tensor:
        return self.raw[:, carl.OBS_BALL + carl.STATE_PER_CAR * self.n_cars:]

    @property
    def boost_pad_active(self) -> th.Tensor:
        return self.boost_pad_values.bool()


@dataclass(frozen=True)
class CarlEvents:
    score_delta: th.Tensor
    done: th.Tensor
    terminated: th.Tensor
    truncated: th.Tensor


@dataclass(frozen=True)
class RewardContext:
    current: CarlState
    previous: CarlState
    current_observation: CARLObservation
    previous_observation: CARLObservation
    events: CarlEvents
    actions: th.Tensor
    score_difference: th.Tensor
    episode_ticks: th.Tensor
    overtime: th.Tensor


__all__ = [
    "BOOST_PAD_POSITIONS",
    "CARLBall",
    "CARLCar",
    "CARLCars",
    "CARLMatchReset",
    "CARLObservation",
    "CARLResetState",
    "REGULATION_TICKS",
    "CarlEvents",
    "CarlState",
    "RewardContext",
]
