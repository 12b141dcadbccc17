"""Named views over the packed observation and state rows, and the records
the vector environment passes to reward functions and reset providers.

Interface (class names, attribute names, the slices they return, the
reset-state contract): python/carl/gymnasium/state.py:10-530.  Column
positions come from the native module's constants, which restate the layout
of include/Cuda/DLPack.h:60-107.

Every named view is a descriptor generated from one of three field tables
(car, ball, observation row), so each layout is written down once and every
view is a slice that shares storage with the packed tensor.
"""
from __future__ import annotations

import functools
from collections.abc import Mapping
from dataclasses import dataclass, field
from typing import Any, NamedTuple

import torch as th

import carl_amd as carl
from carl_amd import BOOST_PAD_POSITIONS, REGULATION_TICKS


class _Cols:
    """Descriptor: columns [start, stop) of the last axis, or column `start`
    alone when stop is None (as bool when `flag`).  `via` names an attribute
    of the owner whose value is sliced instead of the owner itself."""

    def __init__(self, start: int, stop: int | None = None, *, flag: bool = False, via: str | None = None,
                 doc: str = ""):
        self.start, self.stop, self.flag, self.via = start, stop, flag, via
        self.__doc__ = doc

    def __get__(self, obj, owner=None):
        if obj is None:
            return self
        base = getattr(obj, self.via) if self.via else obj
        cols = base[..., self.start] if self.stop is None else base[..., self.start:self.stop]
        return cols.bool() if self.flag else cols


class _Field(NamedTuple):
    name: str
    start: int
    stop: int | None
    flag: bool
    doc: str


# columns of one car (observation car block; the canonical state's car rows
# carry the same columns plus the ball-touch flag)
_PHYSICS_FIELDS = (
    _Field("position", carl.OBS_POS, carl.OBS_VEL, False, "position (uu)"),
    _Field("velocity", carl.OBS_VEL, carl.OBS_ANG, False, "linear velocity (uu/s)"),
    _Field("angular_velocity", carl.OBS_ANG, carl.OBS_FORWARD, False, "angular velocity (rad/s)"),
)
_CAR_FIELDS = _PHYSICS_FIELDS + (
    _Field("forward", carl.OBS_FORWARD, carl.OBS_UP, False, "unit forward axis"),
    _Field("up", carl.OBS_UP, carl.OBS_BOOST, False, "unit up axis"),
    _Field("boost", carl.OBS_BOOST, None, False, "boost amount [0, 100]"),
    _Field("on_ground", carl.OBS_ON_GROUND, None, True, "three or more wheels touching"),
    _Field("demoed", carl.OBS_DEMOED, None, True, "demolished, waiting to respawn"),
    _Field("has_flipped", carl.OBS_HAS_FLIPPED, None, True, "the flip of this jump is used"),
    _Field("has_double_jumped", carl.OBS_HAS_DOUBLE_JUMPED, None, True, "the double jump is used"),
    _Field("is_boosting", carl.OBS_IS_BOOSTING, None, True, "boosting this tick"),
)


def _install(cls, fields, *, prefix: str = "", via: str | None = None):
    for f in fields:
        setattr(cls, prefix + f.name, _Cols(f.start, f.stop, flag=f.flag, via=via, doc=f.doc))
    return cls


class _Packed(th.Tensor):
    """Tensor subclass whose torch operations return plain tensors; only the
    named views keep the subclass."""

    @classmethod
    def from_tensor(cls, tensor: th.Tensor):
        return tensor.as_subclass(cls)

    @classmethod
    def __torch_function__(cls, func, types, args=(), kwargs=None):
        with th._C.DisableTorchFunctionSubclass():
            return func(*args, **(kwargs or {}))


@functools.partial(_install, fields=_PHYSICS_FIELDS)
class CARLBall(_Packed):
    """[..., OBS_BALL] ball columns: position, velocity, angular velocity."""


@functools.partial(_install, fields=_CAR_FIELDS)
class CARLCar(_Packed):
    """[..., OBS_PER_CAR] columns of one car."""


class CARLCars(CARLCar):
    """[..., n_cars, OBS_PER_CAR]: every car of an observation, the observer
    first, then its teammates, then the opponents."""

    _n_cars: int

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


_install(CARLCars, [f for f in _CAR_FIELDS if f.name in ("position", "velocity", "angular_velocity", "forward",
                                                          "up", "boost")], prefix="ego_", via="ego")


class _ObsColumns(NamedTuple):
    """Start columns of the blocks of an observation row with n cars."""
    car_end: int
    pads_active: int
    pads_distance: int
    ego_ball: int
    others: int
    own_goal: int
    opponent_goal: int
    dodge: int
    controller: int
    previous: int


@functools.lru_cache(maxsize=None)
def _obs_columns(n_cars: int) -> _ObsColumns:
    car_end = carl.OBS_BALL + carl.OBS_PER_CAR * n_cars
    ego_ball = car_end + carl.OBS_BOOST_PADS
    others = ego_ball + carl.OBS_RELATIVE_EGO_BALL
    own_goal = others + carl.OBS_RELATIVE_PER_OTHER_CAR * (n_cars - 1)
    dodge = own_goal + carl.OBS_RELATIVE_GOALS
    controller = dodge + carl.OBS_EGO_DODGE
    return _ObsColumns(car_end=car_end, pads_active=car_end, pads_distance=car_end + carl.NUM_BOOST_PADS,
                       ego_ball=ego_ball, others=others, own_goal=own_goal,
                       opponent_goal=own_goal + carl.OBS_VECTOR_SIZE, dodge=dodge, controller=controller,
                       previous=controller + carl.OBS_EGO_CONTROLLER)


class CARLObservation(_Packed):
    """Observation rows [..., obs_dim] with named views of the packed layout:
    ball, cars, boost pads, relative vectors, goals, dodge window,
    controller state and the optional previous controls."""

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
    def _cols(self) -> _ObsColumns:
        return _obs_columns(self._n_cars)

    def _block(self, start: int, width: int) -> th.Tensor:
        return self[..., start:start + width]

    @property
    def car_end(self) -> int:
        return self._cols.car_end

    @property
    def ball(self) -> CARLBall:
        return CARLBall.from_tensor(self[..., :carl.OBS_BALL])

    @property
    def cars(self) -> CARLCars:
        block = self[..., carl.OBS_BALL:self._cols.car_end]
        return CARLCars.from_tensor(block.view(*self.shape[:-1], self._n_cars, carl.OBS_PER_CAR), self._n_cars)

    ball_values = property(lambda self: self.ball)
    car_values = property(lambda self: self.cars)
    ego_values = property(lambda self: self.cars.ego)

    @property
    def boost_pad_active(self) -> th.Tensor:
        return self._block(self._cols.pads_active, carl.NUM_BOOST_PADS).bool()

    @property
    def boost_pad_distance(self) -> th.Tensor:
        return self._block(self._cols.pads_distance, carl.NUM_BOOST_PADS)

    @property
    def ego_ball_relative(self) -> th.Tensor:
        return self._block(self._cols.ego_ball, carl.OBS_RELATIVE_EGO_BALL)

    @property
    def ego_other_relative(self) -> th.Tensor:
        others = self._n_cars - 1
        block = self._block(self._cols.others, carl.OBS_RELATIVE_PER_OTHER_CAR * others)
        return block.view(*self.shape[:-1], others, carl.OBS_RELATIVE_PER_OTHER_CAR)

    @property
    def own_goal_relative(self) -> th.Tensor:
        return self._block(self._cols.own_goal, carl.OBS_VECTOR_SIZE)

    @property
    def opponent_goal_relative(self) -> th.Tensor:
        return self._block(self._cols.opponent_goal, carl.OBS_VECTOR_SIZE)

    @property
    def ego_has_flip_or_jump(self) -> th.Tensor:
        return self[..., self._cols.dodge].bool()

    @property
    def ego_flip_window_remaining(self) -> th.Tensor:
        return self[..., self._cols.dodge + 1]

    @property
    def ego_controller(self) -> th.Tensor:
        cols = self._cols
        if self.shape[-1] not in (cols.previous, cols.previous + carl.OBS_PREVIOUS_CONTROLS):
            raise ValueError("observation does not match ego controller v3")
        return self[..., cols.controller:cols.previous]

    @property
    def ego_previous_controls(self) -> th.Tensor:
        cols = self._cols
        if self.shape[-1] != cols.previous + carl.OBS_PREVIOUS_CONTROLS:
            if self.shape[-1] != cols.previous:
                raise ValueError("observation does not match ego controller v3")
            raise ValueError("observation does not include previous controls")
        return self[..., cols.previous:]


_install(CARLObservation, _PHYSICS_FIELDS, prefix="ball_", via="ball")
_install(CARLObservation, _CAR_FIELDS, prefix="car_", via="cars")
_install(CARLObservation, (
    _Field("has_jumped", 0, None, True, "jumped since the last landing"),
    _Field("is_jumping", 1, None, True, "jump impulse still applied"),
    _Field("is_flipping", 2, None, True, "a flip is in progress"),
    _Field("flip_time", 3, None, False, "seconds since the flip started"),
    _Field("demo_respawn_time", 4, None, False, "seconds until the respawn"),
), prefix="ego_", via="ego_controller")


@dataclass(frozen=True)
class CARLMatchReset:
    """Scores and episode clock for the simulations a reset restores."""

    blue_score: th.Tensor
    orange_score: th.Tensor
    episode_ticks: th.Tensor


def _column_scale(pairs) -> tuple[float, ...]:
    """Per-column factors from (width, factor or factors) runs."""
    out: list[float] = []
    for width, factor in pairs:
        out.extend(factor if isinstance(factor, tuple) else (factor,) * width)
    return tuple(out)


# normalised -> physics units, column by column (1 where no normalisation applies)
_BALL_SCALE = _column_scale(((3, tuple(carl.OBS_POSITION_SCALE)), (3, carl.BALL_MAX_SPEED),
                             (3, carl.BALL_MAX_ANG_SPEED)))
_CAR_SCALE = _column_scale(((3, tuple(carl.OBS_POSITION_SCALE)), (3, carl.CAR_MAX_SPEED),
                            (3, carl.CAR_MAX_ANG_SPEED), (carl.OBS_BOOST - carl.OBS_FORWARD, 1.0),
                            (1, carl.BOOST_MAX), (carl.OBS_PER_CAR - carl.OBS_BOOST - 1, 1.0)))
assert len(_BALL_SCALE) == carl.OBS_BALL and len(_CAR_SCALE) == carl.OBS_PER_CAR


def _is_arena_mask(mask: th.Tensor, eligible: th.Tensor) -> bool:
    return mask.shape == eligible.shape and mask.dtype == th.bool and mask.device == eligible.device


def _check_indices(indices: th.Tensor | None, eligible: th.Tensor) -> None:
    """Indexed selection: int64 vector on the environment's device, in range,
    without repeats, naming only arenas that are eligible for a reset."""
    if indices is None or indices.ndim != 1 or indices.dtype != th.int64 or indices.device != eligible.device:
        raise ValueError("simulation_indices must be int64 on the environment device")
    n = len(eligible)
    if indices.numel() == 0:
        return
    if int(indices.min()) < 0 or int(indices.max()) >= n:
        raise ValueError("simulation_indices are out of range")
    hits = th.bincount(indices, minlength=n)
    if bool((hits > 1).any()) or bool((hits.bool() & ~eligible).any()):
        raise ValueError("simulation_indices must be unique and selected for reset")


@dataclass(frozen=True)
class CARLResetState:
    """State a reset provider returns, in physics units, or in the
    observation's normalised units when `normalized`.

    Either `simulation_indices` (int64) names one row per restored arena, or
    `simulation_indices` is None and the bool `reset_mask` [n_sim] selects
    arenas from full-size rows; that fixed-shape form is validated from its
    metadata only (no host readback), so its rotations must be valid.
    """

    simulation_indices: th.Tensor | None
    ball: CARLBall
    cars: CARLCars
    car_internal_state: th.Tensor | None = None
    match: CARLMatchReset | None = None
    normalized: bool = False
    reset_mask: th.Tensor | None = None

    def _rows(self, eligible: th.Tensor) -> int:
        if self.reset_mask is None:
            _check_indices(self.simulation_indices, eligible)
            return len(self.simulation_indices)
        if self.simulation_indices is not None:
            raise ValueError("specify reset_mask or simulation_indices, not both")
        if not _is_arena_mask(self.reset_mask, eligible):
            raise ValueError("reset_mask must be bool [n_sim] on the environment device")
        return len(eligible)

    def validate(self, reset_mask: th.Tensor, n_cars: int) -> None:
        rows = self._rows(reset_mask)
        want = ((rows, carl.OBS_BALL), (rows, n_cars, carl.OBS_PER_CAR))
        if (tuple(self.ball.shape), tuple(self.cars.shape)) != want:
            raise ValueError("ball or cars have the wrong shape")

    def physical(self) -> tuple[CARLBall, CARLCars]:
        if not self.normalized:
            return self.ball, self.cars
        ball = CARLBall.from_tensor(self.ball * self.ball.new_tensor(_BALL_SCALE))
        cars = CARLCars.from_tensor(self.cars * self.cars.new_tensor(_CAR_SCALE), self.cars.n_cars)
        return ball, cars


def _state_width(n_cars: int) -> int:
    return carl.OBS_BALL + carl.STATE_PER_CAR * n_cars + carl.NUM_BOOST_PADS


@dataclass(frozen=True)
class CarlState:
    """Canonical (never mirrored) state rows [n_sim, state_dim]: the ball,
    every car in simulation order, then the boost pads."""

    raw: th.Tensor
    n_cars: int
    boost_pad_positions: th.Tensor
    team_sign: th.Tensor

    @classmethod
    def from_raw(cls, raw: th.Tensor, n_cars: int, boost_pad_positions: th.Tensor,
                 team_sign: th.Tensor) -> "CarlState":
        width = _state_width(n_cars)
        if raw.ndim != 2 or raw.shape[1] != width:
            raise ValueError(f"Expected raw state shaped [n_sim, {width}], got {tuple(raw.shape)}")
        return cls(raw, n_cars, boost_pad_positions, team_sign)

    @property
    def ball_values(self) -> th.Tensor:
        return self.raw[:, :carl.OBS_BALL]

    @property
    def car_values(self) -> th.Tensor:
        block = self.raw[:, carl.OBS_BALL:carl.OBS_BALL + carl.STATE_PER_CAR * self.n_cars]
        return block.view(self.raw.shape[0], self.n_cars, carl.STATE_PER_CAR)

    @property
    def boost_pad_values(self) -> th.Tensor:
        return self.raw[:, carl.OBS_BALL + carl.STATE_PER_CAR * self.n_cars:]

    @property
    def boost_pad_active(self) -> th.Tensor:
        return self.boost_pad_values.bool()


_install(CarlState, _PHYSICS_FIELDS, prefix="ball_", via="ball_values")
_install(CarlState, _CAR_FIELDS + (
    _Field("ball_touches", carl.STATE_BALL_TOUCH, None, True, "touched the ball within the step"),), prefix="car_",
    via="car_values")


@dataclass(frozen=True, slots=True)
class CarlEvents:
    """Per-arena outcome of the step: score change and how it ended."""

    score_delta: th.Tensor
    done: th.Tensor
    terminated: th.Tensor
    truncated: th.Tensor


@dataclass(frozen=True, slots=True)
class RewardContext:
    """Everything a reward function sees for one step: the state before and
    after it (`current` is the transition state, before any reset), the
    observations around it, the step's events and actions, and the match
    state at the end of the step."""

    current: CarlState
    previous: CarlState
    current_observation: CARLObservation
    previous_observation: CARLObservation
    events: CarlEvents
    actions: th.Tensor
    score_difference: th.Tensor
    episode_ticks: th.Tensor
    overtime: th.Tensor


@dataclass(frozen=True)
class RewardResult:
    """A reward function's [n_sim, n_cars] reward plus info entries."""

    reward: th.Tensor
    info: Mapping[str, list[Any]] = field(default_factory=dict)


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
