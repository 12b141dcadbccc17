"""Torch vector environment over the MI355X engine.

Interface and behaviour: python/carl/gymnasium/torch.py:79-605
(CARLTorchVectorEnv): Gymnasium SAME_STEP autoreset (arenas that finish are
reset inside step(); terminated = finished with a goal, truncated = finished
otherwise), the default reward (score change x team sign) or the sum of
registered reward functions over a RewardContext, optional reset-state
providers (indexed, or fixed-shape with a mask and no host readback), and
episode return/length reports, immediate or deferred to a rollout boundary.

Structure: the environment composes three parts:
  * `_StreamBridge` orders torch's current stream and the engine's private
    stream around every native call;
  * `_request_from_typed` / `_request_from_mapping` turn what a reset
    provider returned (a CARLResetState or a mapping of tensors) into the
    arguments of one `Env.apply_reset_state` call, or into none;
  * `_EpisodeLedger` keeps the per-agent returns and lengths and produces the
    episode reports.
"""
from __future__ import annotations

import math
from collections.abc import Callable, Iterable, Mapping
from typing import Any, NamedTuple

import numpy as np
import torch as th
import torch.nn.functional as F

import carl_amd as carl

from ._compat import AutoresetMode, Box, MultiDiscrete, VectorEnv, batch_space
from .action import CARLActionCodec
from .state import (
    BOOST_PAD_POSITIONS,
    REGULATION_TICKS,
    CARLObservation,
    CARLResetState,
    CarlEvents,
    CarlState,
    RewardContext,
    RewardResult,
)

RewardFunction = Callable[[RewardContext], "th.Tensor | RewardResult"]
ResetState = "CARLResetState | Mapping[str, th.Tensor]"
ResetStateProvider = Callable[[th.Tensor], Any]


# --------------------------------------------------------------- rotations

def _forward_up_to_quat(forward: th.Tensor, up: th.Tensor, *, validate: bool = True) -> th.Tensor:
    """Unit quaternions [x, y, z, w] of the car frames whose local x axis is
    `forward` and local z axis is `up` (re-orthonormalised: right =
    up x forward, both normalised, then up = forward x right).

    The conversion takes each component's magnitude from the square root of
    its diagonal combination of the rotation matrix R and the signs of x, y
    and z from the antisymmetric part (the copysign form of the
    matrix-to-quaternion conversion; w >= 0), then normalises.  These are the
    float operations, in the same order, of the reference's conversion
    (python/carl/gymnasium/torch.py:31-61), so a restored rotation is the
    reference's bit for bit; on a frame with up = +z the x and y components
    are the square roots of the rounding residue of 1 + R00 - R11 - R22 (up to
    about 3e-4), as in the reference, not exactly 0."""
    right = th.linalg.cross(up, forward, dim=-1)
    if validate:
        if not (th.isfinite(forward).all() and th.isfinite(up).all()):
            raise ValueError("car forward and up directions must be finite")
        degenerate = (forward * forward).sum(-1).lt(1e-8) | (right * right).sum(-1).lt(1e-8)
        if degenerate.any():
            raise ValueError("car forward and up directions must define a rotation")
    ex = F.normalize(forward, dim=-1)
    ey = F.normalize(right, dim=-1)
    ez = th.linalg.cross(ex, ey, dim=-1)
    # R = [ex ey ez] (columns): R[i][j] is component i of column j
    r00, r11, r22 = ex[..., 0], ey[..., 1], ez[..., 2]
    diag = (
        1 + r00 + r11 + r22,      # 4 w^2
        1 + r00 - r11 - r22,      # 4 x^2
        1 - r00 + r11 - r22,      # 4 y^2
        1 - r00 - r11 + r22,      # 4 z^2
    )
    mags = [d.clamp_min(0).sqrt() for d in diag]
    signs = (ey[..., 2] - ez[..., 1], ez[..., 0] - ex[..., 2], ex[..., 1] - ey[..., 0])   # 4wx, 4wy, 4wz
    wxyz = th.stack([mags[0]] + [th.copysign(m, sg) for m, sg in zip(mags[1:], signs)], dim=-1)
    return F.normalize(wxyz, dim=-1)[..., (1, 2, 3, 0)]


def _ticks(ticks: int | None, seconds: float | None, default: int | None) -> int | None:
    """A timeout given in ticks or in seconds (rounded up to whole ticks)."""
    if ticks is not None and seconds is not None:
        raise ValueError("Specify ticks or seconds, not both")
    if seconds is not None:
        if not (math.isfinite(seconds) and seconds > 0):
            raise ValueError("Timeout seconds must be positive and finite")
        ticks = math.ceil(seconds * carl.PHYS_TICKS_PER_SECOND)
    if ticks is None:
        return default
    if ticks < 1:
        raise ValueError("Timeout ticks must be positive")
    return ticks


# ----------------------------------------------------------------- streams

class _StreamBridge:
    """Orders work between the caller's current torch stream and the
    engine's stream: both wait for each other (or, with `synchronize`, the
    whole device is synchronised)."""

    def __init__(self, handle: int, device: th.device, synchronize: bool):
        self.device = device
        self.synchronize = synchronize
        self.engine = th.cuda.ExternalStream(handle, device=device)

    def join(self) -> None:
        if self.synchronize:
            th.cuda.synchronize(self.device)
            return
        caller = th.cuda.current_stream(self.device)
        self.engine.wait_stream(caller)
        caller.wait_stream(self.engine)


# ------------------------------------------------------------------ resets

_REQUIRED = ("ball_position", "ball_velocity", "ball_angular_velocity", "car_position", "car_rotation",
             "car_velocity", "car_angular_velocity", "car_demoed")
_OPTIONAL = ("car_boost", "car_internal_state", "blue_score", "orange_score", "episode_ticks")


class _ResetRequest(NamedTuple):
    """Arguments of one Env.apply_reset_state call."""
    required: tuple[th.Tensor, ...]      # in _REQUIRED order
    optional: dict[str, th.Tensor | None]
    indices: th.Tensor | None
    mask: th.Tensor | None


def _contiguous(x: th.Tensor | None) -> th.Tensor | None:
    return None if x is None else x.contiguous()


def _arena_selection(mask: th.Tensor, eligible: th.Tensor) -> th.Tensor:
    """A provider's mask restricted to the arenas eligible for a reset."""
    if mask.shape != (len(eligible),) or mask.dtype != th.bool or mask.device != eligible.device:
        raise ValueError("reset_mask must be bool [n_sim] on the environment device")
    return (mask & eligible).contiguous()


def _request_from_mapping(state: Mapping[str, th.Tensor], eligible: th.Tensor,
                          masked_only: bool) -> _ResetRequest | None:
    if "reset_mask" in state:
        if "simulation_indices" in state:
            raise ValueError("specify reset_mask or simulation_indices, not both")
        indices, mask = None, _arena_selection(state["reset_mask"], eligible)
    else:
        if masked_only:
            raise ValueError("masked reset providers must supply reset_mask")
        indices = state.get("simulation_indices")
        if indices is None:
            indices = eligible.nonzero(as_tuple=True)[0]
        if indices.numel() == 0:
            return None
        indices, mask = indices.contiguous(), None
    return _ResetRequest(tuple(state[k].contiguous() for k in _REQUIRED),
                         {k: _contiguous(state.get(k)) for k in _OPTIONAL}, indices, mask)


def _request_from_typed(state: CARLResetState, eligible: th.Tensor, n_cars: int,
                        masked_only: bool) -> _ResetRequest | None:
    masked = state.reset_mask is not None
    if masked_only and not masked:
        raise ValueError("masked reset providers must supply reset_mask")
    state.validate(eligible, n_cars)
    if not masked and state.simulation_indices.numel() == 0:
        return None
    ball, cars = state.physical()
    # fixed-shape requests stay on the device: no host-side rotation check
    rotation = _forward_up_to_quat(cars.forward, cars.up, validate=not masked).contiguous()
    required = (ball.position, ball.velocity, ball.angular_velocity, cars.position, rotation, cars.velocity,
                cars.angular_velocity, cars.demoed)
    match = state.match
    optional = {
        "car_boost": cars.boost,
        "car_internal_state": state.car_internal_state,
        "blue_score": None if match is None else match.blue_score,
        "orange_score": None if match is None else match.orange_score,
        "episode_ticks": None if match is None else match.episode_ticks,
    }
    return _ResetRequest(tuple(x.contiguous() for x in required), {k: _contiguous(v) for k, v in optional.items()},
                         None if masked else state.simulation_indices.contiguous(),
                         _arena_selection(state.reset_mask, eligible) if masked else None)


# ---------------------------------------------------------------- episodes

class _EpisodeLedger:
    """Running return and length per agent, and the reports of episodes that
    end: returned by the step that ends them, or (deferred) kept on the
    device until drained, in step and agent order."""

    def __init__(self, n_envs: int, device: th.device, deferred: bool):
        self.deferred = deferred
        self.returns = th.zeros(n_envs, device=device)
        self.lengths = th.zeros(n_envs, dtype=th.int64, device=device)
        self.pending: list[tuple[th.Tensor, th.Tensor, th.Tensor]] = []

    def clear(self) -> None:
        self.returns.zero_()
        self.lengths.zero_()
        self.pending.clear()

    def record(self, reward: th.Tensor, done: th.Tensor) -> dict[str, list[Any]] | None:
        """Add a step; the report of the episodes it ends (None if none
        ended or reports are deferred)."""
        self.returns += reward
        self.lengths += 1
        if self.deferred:
            self.pending.append((self.returns.clone(), self.lengths.clone(), done.clone()))
            self.returns.masked_fill_(done, 0)
            self.lengths.masked_fill_(done, 0)
            return None
        ended = done.nonzero(as_tuple=True)[0]
        if ended.numel() == 0:
            return None
        report = {"reward": self.returns[ended].cpu().tolist(), "length": self.lengths[ended].cpu().tolist()}
        self.returns[ended] = 0
        self.lengths[ended] = 0
        return report

    def drain(self) -> dict[str, list[Any]]:
        if not self.pending:
            return {"reward": [], "length": []}
        returns, lengths, dones = (th.stack(x).flatten() for x in zip(*self.pending))
        ended = dones.nonzero(as_tuple=True)[0]
        self.pending.clear()
        return {"reward": returns[ended].cpu().tolist(), "length": lengths[ended].cpu().tolist()}


# ----------------------------------------------------------- environment

class CARLTorchVectorEnv(VectorEnv):
    """Torch vector environment, one agent per car of every arena.

    With ``masked_resets=True`` the reset provider is called on every step,
    also when no arena finished, and must return full-size tensors with a
    ``reset_mask`` (CARLResetState or mapping); the selection stays on the
    GPU.  Providers may return None.  Input storage must stay unchanged until
    the engine's stream has read it.
    """

    metadata = {"render_modes": [], "autoreset_mode": AutoresetMode.SAME_STEP}
    render_mode = spec = None

    def __init__(
        self,
        n_sim: int,
        n_blue: int,
        n_orange: int,
        seed: int = 0,
        frameskip: int = 8,
        max_ticks: int = REGULATION_TICKS,
        *,
        overtime_timeout_ticks: int | None = None,
        overtime_timeout_seconds: float | None = None,
        no_touch_timeout_ticks: int | None = None,
        no_touch_timeout_seconds: float | None = None,
        invert_orange: bool = True,
        normalize: bool = False,
        previous_controls: bool = False,
        copy_outputs: bool = True,
        synchronize: bool = False,
        reward_funcs: Iterable[RewardFunction] | None = None,
        reward_scale: float = 1.0,
        reset_state_provider: ResetStateProvider | None = None,
        masked_resets: bool = False,
        defer_episode_reporting: bool = False,
        discrete_actions: bool = False,
    ) -> None:
        super().__init__()
        if max_ticks < 1 or reward_scale <= 0:
            raise ValueError("max_ticks and reward_scale must be positive")
        overtime = _ticks(overtime_timeout_ticks, overtime_timeout_seconds, REGULATION_TICKS)
        no_touch = _ticks(no_touch_timeout_ticks, no_touch_timeout_seconds, 0)

        self.device = th.device("cuda:0")
        self.closed = False
        self.reward_funcs = list(reward_funcs or ())
        self.reward_scale = reward_scale
        self.reset_state_provider = reset_state_provider
        self.masked_resets = masked_resets
        self.defer_episode_reporting = defer_episode_reporting
        self.discrete_actions = discrete_actions
        self._seed = seed
        self._copy_outputs = copy_outputs

        env = carl.Env(n_sim=n_sim, n_blue=n_blue, n_orange=n_orange, seed=seed, frameskip=frameskip,
                       invert_orange=invert_orange, normalize=normalize, previous_controls=previous_controls)
        env.max_ticks = max_ticks
        env.overtime_timeout_ticks = overtime
        env.no_touch_timeout_ticks = no_touch
        self._env = env
        self._bridge = _StreamBridge(env.stream, self.device, synchronize)

        self.n_sim = n_sim
        self.n_cars = env.n_cars
        self.n_envs = n_sim * self.n_cars
        self._obs_dim = env.obs_dim
        self._team_sign = th.tensor([1.0] * n_blue + [-1.0] * n_orange, device=self.device)
        self._pad_positions = th.tensor(BOOST_PAD_POSITIONS, dtype=th.float32, device=self.device)
        self.action_codec = CARLActionCodec(previous_controls).to(self.device) if discrete_actions else None
        self._ledger = _EpisodeLedger(self.n_envs, self.device, defer_episode_reporting)

        # match state at the end of the last step (reward context), cleared
        # for the arenas that reset
        self._score_difference = th.zeros(n_sim, dtype=th.int32, device=self.device)
        self._episode_ticks = th.zeros(n_sim, dtype=th.int32, device=self.device)
        self._overtime = th.zeros(n_sim, dtype=th.bool, device=self.device)
        # state and observation after the last step or reset (reward context)
        self._state: CarlState | None = None
        self._observation: CARLObservation | None = None

        self.single_observation_space = Box(-np.inf, np.inf, (self._obs_dim,), np.float32)
        if discrete_actions:
            self.single_action_space = MultiDiscrete(np.asarray(carl.ACTION_NVECS, dtype=np.int64))
        else:
            self.single_action_space = Box(np.asarray(carl.CONTINUOUS_ACTION_LOW, dtype=np.float32),
                                           np.asarray(carl.CONTINUOUS_ACTION_HIGH, dtype=np.float32))
        self.observation_space = batch_space(self.single_observation_space, self.n_envs)
        self.action_space = batch_space(self.single_action_space, self.n_envs)

    # -- native outputs

    def _read(self, capsule: object, copy: bool | None = None) -> th.Tensor:
        """An engine output as a tensor: a copy, or (copy_outputs=False) a
        view that the engine rewrites on its next call."""
        x = th.from_dlpack(capsule)
        return x.clone() if (self._copy_outputs if copy is None else copy) else x

    def _obs_view(self, capsule: object) -> CARLObservation:
        return CARLObservation.from_tensor(self._read(capsule).view(self.n_envs, self._obs_dim), self.n_cars)

    def _canonical(self, capsule: object) -> CarlState:
        return CarlState.from_raw(self._read(capsule, copy=True), self.n_cars, self._pad_positions, self._team_sign)

    def _observe(self) -> CARLObservation:
        self._bridge.join()
        obs = self._obs_view(self._env.get_obs())
        keep = bool(self.reward_funcs)
        self._state = self._canonical(self._env.get_state()) if keep else None
        self._observation = obs if keep else None
        return obs

    def _agents(self, per_arena: th.Tensor) -> th.Tensor:
        """[n_sim] -> [n_envs], one entry per car."""
        return per_arena.repeat_interleave(self.n_cars)

    def _ensure_open(self) -> None:
        if self.closed:
            raise RuntimeError("Environment is closed")

    # -- resets

    def _apply_reset_state(self, reset_mask: th.Tensor) -> None:
        """Run the reset provider for the arenas in `reset_mask` (bool
        [n_sim]) and apply what it returns."""
        provider = self.reset_state_provider
        if provider is None or not (self.masked_resets or reset_mask.any()):
            return
        state = provider(reset_mask)
        if state is None:
            return
        if isinstance(state, CARLResetState):
            request = _request_from_typed(state, reset_mask, self.n_cars, self.masked_resets)
        else:
            request = _request_from_mapping(state, reset_mask, self.masked_resets)
        if request is None:
            return
        self._env.apply_reset_state(*request.required, **request.optional,
                                    simulation_indices=request.indices, reset_mask=request.mask)

    def _forget_match(self, arenas: th.Tensor) -> None:
        self._score_difference.masked_fill_(arenas, 0)
        self._episode_ticks.masked_fill_(arenas, 0)
        self._overtime.masked_fill_(arenas, False)

    # -- rewards

    def register_reward(self, reward_function: RewardFunction) -> RewardFunction:
        self.reward_funcs.append(reward_function)
        return reward_function

    def action_mask(self, observation: th.Tensor) -> th.Tensor:
        if self.action_codec is None:
            raise RuntimeError("continuous controls do not use a categorical action mask")
        return self.action_codec.mask(observation)

    def _reward_context(self, actions: th.Tensor, events: CarlEvents) -> RewardContext:
        if self._state is None or self._observation is None:
            raise RuntimeError("reset must be called before using custom rewards")
        return RewardContext(
            current=self._canonical(self._env.get_transition_state()),
            previous=self._state,
            current_observation=self._obs_view(self._env.get_obs()),
            previous_observation=self._observation,
            events=events,
            actions=actions,
            score_difference=self._score_difference,
            episode_ticks=self._episode_ticks,
            overtime=self._overtime,
        )

    def _custom_reward(self, actions: th.Tensor, events: CarlEvents) -> tuple[th.Tensor, dict[str, list[Any]]]:
        context = self._reward_context(actions, events)
        total = th.zeros((self.n_sim, self.n_cars), device=self.device)
        info: dict[str, list[Any]] = {}
        for func in self.reward_funcs:
            out = func(context)
            if isinstance(out, RewardResult):
                info.update(out.info)
                out = out.reward
            if out.shape != total.shape:
                raise ValueError(f"Reward must have shape {tuple(total.shape)}")
            total += out
        return (total * self.reward_scale).reshape(self.n_envs), info

    # -- gymnasium API

    def reset(self, *, seed: int | None = None, options: dict[str, Any] | None = None) -> th.Tensor:
        self._ensure_open()
        if seed is not None and seed != self._seed:
            raise ValueError("CARL's seed is constructor-only")
        if options:
            raise NotImplementedError("CARL reset options are not supported")
        self._bridge.join()
        self._env.reset()
        self._apply_reset_state(th.ones(self.n_sim, dtype=th.bool, device=self.device))
        self._ledger.clear()
        for x in (self._score_difference, self._episode_ticks, self._overtime):
            x.zero_()
        return self._observe()

    def set_ball(self, position: th.Tensor, velocity: th.Tensor, angular_velocity: th.Tensor, *,
                 simulation_indices: th.Tensor | None = None) -> th.Tensor:
        self._ensure_open()
        self._bridge.join()
        self._env.set_ball(position.contiguous(), velocity.contiguous(), angular_velocity.contiguous(),
                           simulation_indices=_contiguous(simulation_indices))
        return self._observe()

    def set_car(self, position: th.Tensor, rotation: th.Tensor, velocity: th.Tensor, angular_velocity: th.Tensor,
                demoed: th.Tensor, *, boost: th.Tensor | None = None, internal_state: th.Tensor | None = None,
                simulation_indices: th.Tensor | None = None) -> th.Tensor:
        self._ensure_open()
        self._bridge.join()
        self._env.set_car(position.contiguous(), rotation.contiguous(), velocity.contiguous(),
                          angular_velocity.contiguous(), demoed.contiguous(), boost=_contiguous(boost),
                          internal_state=_contiguous(internal_state),
                          simulation_indices=_contiguous(simulation_indices))
        return self._observe()

    def step(self, actions: th.Tensor | np.ndarray):
        self._ensure_open()
        width = len(carl.ACTION_NVECS)
        actions = th.as_tensor(actions, dtype=th.int32 if self.discrete_actions else th.float32,
                               device=self.device).contiguous()
        if actions.shape != (self.n_envs, width):
            raise ValueError(f"Expected actions shaped {(self.n_envs, width)}")
        actions = actions.view(self.n_sim, self.n_cars, width)

        self._bridge.join()
        (self._env.step if self.discrete_actions else self._env.step_continuous)(actions)
        self._bridge.join()

        env = self._env
        score_delta = self._read(env.get_rewards())
        finished = self._read(env.get_dones())
        self._score_difference = self._read(env.get_transition_score_difference())
        self._episode_ticks = self._read(env.get_transition_episode_ticks())
        self._overtime = self._read(env.get_transition_overtime())
        goal = finished & (score_delta != 0)
        events = CarlEvents(score_delta=score_delta, done=finished, terminated=goal, truncated=finished & ~goal)

        if self.reward_funcs:
            reward, reward_info = self._custom_reward(actions, events)
        else:
            reward, reward_info = (score_delta[:, None] * self._team_sign).reshape(self.n_envs), {}

        self._apply_reset_state(finished)
        self._forget_match(finished)
        obs = self._observe()

        terminated, truncated = self._agents(events.terminated), self._agents(events.truncated)
        done = terminated | truncated
        report = self._ledger.record(reward, done)
        if self.defer_episode_reporting:
            info = {**reward_info, "final_obs": self._obs_view(env.get_transition_obs()), "_final_obs": done}
        elif report is None:
            info = {"reward": [], "length": []}
        else:
            info = {**report, "final_obs": self._obs_view(env.get_transition_obs()), "_final_obs": done,
                    **reward_info}
        return obs, reward, terminated, truncated, info

    def drain_episode_reports(self) -> dict[str, list[Any]]:
        """Reports of every episode that ended since the last drain, in step
        and agent order (deferred reporting).  reset() discards them."""
        self._ensure_open()
        return self._ledger.drain()

    def render(self) -> None:
        return None

    def close(self, **_: Any) -> None:
        if self.closed:
            return
        self._bridge.join()
        del self._env
        self.closed = True
