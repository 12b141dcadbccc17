"""Torch vector environment over the MI355X engine.

API- and behaviour-compatible with CARLTorchVectorEnv
(python/carl/gymnasium/torch.py:79-605):
  * Gymnasium SAME_STEP autoreset: finished arenas are reset inside step();
    terminated = done with a goal, truncated = done otherwise;
  * default reward = per-step score delta * team sign, or the sum of
    registered reward functions over a RewardContext;
  * optional reset-state providers, indexed or fixed-shape (masked), applied
    to finished arenas; masked providers never force a host synchronisation;
  * episode return/length reporting, immediate or deferred.
All engine work runs on the environment's private HIP stream; the torch
current stream is joined to it around every native call.
"""
from __future__ import annotations

import math
from collections.abc import Callable, Iterable, Mapping
from typing import Any

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


def _forward_up_to_quat(forward: th.Tensor, up: th.Tensor, *, validate: bool = True) -> th.Tensor:
    """Car axes -> unit quaternions in [x, y, z, w] order.

    The basis is re-orthonormalised (right = up x forward, up = forward x
    right) and converted with the sign-copy form of the matrix-to-quaternion
    map: |q_i| from the diagonal, signs from the antisymmetric parts.
    """
    right = th.linalg.cross(up, forward, dim=-1)
    if validate:
        if not th.isfinite(forward).all() or not th.isfinite(up).all():
            raise ValueError("car forward and up directions must be finite")
        if (forward.square().sum(-1) < 1e-8).any() or (right.square().sum(-1) < 1e-8).any():
            raise ValueError("car forward and up directions must define a rotation")
    f = F.normalize(forward, dim=-1)
    r = F.normalize(right, dim=-1)
    u = th.linalg.cross(f, r, dim=-1)
    m = th.stack((f, r, u), dim=-1)  # columns: forward, right, up
    m00, m11, m22 = m[..., 0, 0], m[..., 1, 1], m[..., 2, 2]
    w = (1 + m00 + m11 + m22).clamp_min(0).sqrt()
    x = th.copysign((1 + m00 - m11 - m22).clamp_min(0).sqrt(), m[..., 2, 1] - m[..., 1, 2])
    y = th.copysign((1 - m00 + m11 - m22).clamp_min(0).sqrt(), m[..., 0, 2] - m[..., 2, 0])
    z = th.copysign((1 - m00 - m11 + m22).clamp_min(0).sqrt(), m[..., 1, 0] - m[..., 0, 1])
    return F.normalize(th.stack((x, y, z, w), dim=-1), dim=-1)


def _ticks(ticks: int | None, seconds: float | None, default: int | None) -> int | None:
    """Resolve a timeout given either in ticks or in seconds."""
    if ticks is not None and seconds is not None:
        raise ValueError("Specify ticks or seconds, not both")
    if seconds is not None:
        if not math.isfinite(seconds) or seconds <= 0:
            raise ValueError("Timeout seconds must be positive and finite")
        ticks = math.ceil(seconds * carl.PHYS_TICKS_PER_SECOND)
    if ticks is not None and ticks < 1:
        raise ValueError("Timeout ticks must be positive")
    return default if ticks is None else ticks


_OPTIONAL_FIELDS = ("car_boost", "car_internal_state", "blue_score", "orange_score", "episode_ticks")


class CARLTorchVectorEnv(VectorEnv):
    """Torch vector environment with optional fixed-shape reset providers.

    ``masked_resets=True`` calls the provider on every step, including when no
    arena is done; it must return full-size tensors and ``reset_mask``.
    Input storage must not be modified until the engine stream has read it.
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

        self.n_sim = n_sim
        self.device = th.device("cuda:0")
        self.closed = False
        self._seed = seed
        self._copy_outputs = copy_outputs
        self._synchronize = synchronize
        self.reward_funcs = list(reward_funcs or ())
        self.reward_scale = reward_scale
        self.reset_state_provider = reset_state_provider
        self.masked_resets = masked_resets
        self.defer_episode_reporting = defer_episode_reporting
        self._episode_reports: list[tuple[th.Tensor, th.Tensor, th.Tensor]] = []
        self.discrete_actions = discrete_actions
        self._state: CarlState | None = None
        self._observation: CARLObservation | None = None

        self._env = carl.Env(n_sim=n_sim, n_blue=n_blue, n_orange=n_orange, seed=seed, frameskip=frameskip,
                             invert_orange=invert_orange, normalize=normalize, previous_controls=previous_controls)
        self._stream = th.cuda.ExternalStream(self._env.stream, device=self.device)
        self._env.max_ticks = max_ticks
        self._env.overtime_timeout_ticks = _ticks(overtime_timeout_ticks, overtime_timeout_seconds, REGULATION_TICKS)
        self._env.no_touch_timeout_ticks = _ticks(no_touch_timeout_ticks, no_touch_timeout_seconds, 0)

        self.n_cars = self._env.n_cars
        self.n_envs = n_sim * self.n_cars
        self._team_sign = th.tensor([1.0] * n_blue + [-1.0] * n_orange, dtype=th.float32, device=self.device)
        self._boost_pad_positions = th.tensor(BOOST_PAD_POSITIONS, dtype=th.float32, device=self.device)
        self.action_codec = (CARLActionCodec(previous_controls=previous_controls).to(self.device)
                             if discrete_actions else None)

        self._episode_return = th.zeros(self.n_envs, device=self.device)
        self._episode_length = th.zeros(self.n_envs, dtype=th.int64, device=self.device)
        self._score_difference = th.zeros(n_sim, dtype=th.int32, device=self.device)
        self._episode_ticks = th.zeros(n_sim, dtype=th.int32, device=self.device)
        self._overtime = th.zeros(n_sim, dtype=th.bool, device=self.device)

        self.single_observation_space = Box(-np.inf, np.inf, (self._env.obs_dim,), np.float32)
        if discrete_actions:
            self.single_action_space = MultiDiscrete(np.asarray(carl.ACTION_NVECS, dtype=np.int64))
        else:
            self.single_action_space = Box(np.asarray(carl.CONTINUOUS_ACTION_LOW, dtype=np.float32),
                                           np.asarray(carl.CONTINUOUS_ACTION_HIGH, dtype=np.float32))
        self.observation_space = batch_space(self.single_observation_space, self.n_envs)
        self.action_space = batch_space(self.single_action_space, self.n_envs)

    # ------------------------------------------------------------- plumbing

    def _check_open(self) -> None:
        if self.closed:
            raise RuntimeError("Environment is closed")

    def _sync(self) -> None:
        if self._synchronize:
            th.cuda.synchronize(self.device)
            return
        current = th.cuda.current_stream(self.device)
        self._stream.wait_stream(current)
        current.wait_stream(self._stream)

    def _tensor(self, capsule: object, *, copy: bool | None = None) -> th.Tensor:
        x = th.from_dlpack(capsule)
        return x.clone() if (self._copy_outputs if copy is None else copy) else x

    def _carl_state(self, capsule: object) -> CarlState:
        return CarlState.from_raw(self._tensor(capsule, copy=True), self.n_cars, self._boost_pad_positions,
                                  self._team_sign)

    def _observation_of(self, capsule: object) -> CARLObservation:
        return CARLObservation.from_tensor(self._tensor(capsule).view(self.n_envs, self._env.obs_dim), self.n_cars)

    def _observe(self) -> CARLObservation:
        self._sync()
        observation = self._observation_of(self._env.get_obs())
        self._state = self._carl_state(self._env.get_state()) if self.reward_funcs else None
        self._observation = observation if self.reward_funcs else None
        return observation

    def _per_car(self, x: th.Tensor) -> th.Tensor:
        return x[:, None].expand(-1, self.n_cars).reshape(self.n_envs)

    # ---------------------------------------------------------- reset states

    def _reset_selection(self, mask: th.Tensor, eligible: th.Tensor) -> th.Tensor:
        if mask.shape != (self.n_sim,) or mask.dtype != th.bool or mask.device != eligible.device:
            raise ValueError("reset_mask must be bool [n_sim] on the environment device")
        return (mask & eligible).contiguous()

    def _apply_reset_state(self, reset_mask: th.Tensor) -> None:
        if self.reset_state_provider is None:
            return
        if not self.masked_resets and not reset_mask.any():
            return
        state = self.reset_state_provider(reset_mask)
        if state is None:
            return
        if isinstance(state, CARLResetState):
            self._apply_typed_reset_state(state, reset_mask)
        else:
            self._apply_mapping_reset_state(state, reset_mask)

    def _apply_mapping_reset_state(self, state: Mapping[str, th.Tensor], reset_mask: th.Tensor) -> None:
        indices = mask = None
        if "reset_mask" in state:
            if "simulation_indices" in state:
                raise ValueError("specify reset_mask or simulation_indices, not both")
            mask = self._reset_selection(state["reset_mask"], reset_mask)
        else:
            if self.masked_resets:
                raise ValueError("masked reset providers must supply reset_mask")
            indices = state.get("simulation_indices")
            if indices is None:
                indices = reset_mask.nonzero(as_tuple=True)[0]
            if not indices.numel():
                return
            indices = indices.contiguous()
        optional = {k: (state[k].contiguous() if k in state else None) for k in _OPTIONAL_FIELDS}
        self._env.apply_reset_state(
            state["ball_position"].contiguous(), state["ball_velocity"].contiguous(),
            state["ball_angular_velocity"].contiguous(), state["car_position"].contiguous(),
            state["car_rotation"].contiguous(), state["car_velocity"].contiguous(),
            state["car_angular_velocity"].contiguous(), state["car_demoed"].contiguous(),
            **optional, simulation_indices=indices, reset_mask=mask)

    def _apply_typed_reset_state(self, state: CARLResetState, reset_mask: th.Tensor) -> None:
        masked = state.reset_mask is not None
        if self.masked_resets and not masked:
            raise ValueError("masked reset providers must supply reset_mask")
        state.validate(reset_mask, self.n_cars)
        if not masked and not state.simulation_indices.numel():
            return
        ball, cars = state.physical()
        rotation = _forward_up_to_quat(cars.forward, cars.up, validate=not masked).contiguous()
        match = state.match
        self._env.apply_reset_state(
            ball.position.contiguous(), ball.velocity.contiguous(), ball.angular_velocity.contiguous(),
            cars.position.contiguous(), rotation, cars.velocity.contiguous(), cars.angular_velocity.contiguous(),
            cars.demoed.contiguous(), car_boost=cars.boost.contiguous(),
            car_internal_state=(state.car_internal_state.contiguous()
                                if state.car_internal_state is not None else None),
            blue_score=match.blue_score.contiguous() if match is not None else None,
            orange_score=match.orange_score.contiguous() if match is not None else None,
            episode_ticks=match.episode_ticks.contiguous() if match is not None else None,
            simulation_indices=None if masked else state.simulation_indices.contiguous(),
            reset_mask=self._reset_selection(state.reset_mask, reset_mask) if masked else None)

    def _clear_sim_stats(self, mask: th.Tensor | None = None) -> None:
        if mask is None:
            self._episode_reports.clear()
            self._episode_return.zero_()
            self._episode_length.zero_()
            self._score_difference.zero_()
            self._episode_ticks.zero_()
            self._overtime.zero_()
            return
        self._score_difference.masked_fill_(mask, 0)
        self._episode_ticks.masked_fill_(mask, 0)
        self._overtime.masked_fill_(mask, False)

    # -------------------------------------------------------------- rewards

    def register_reward(self, reward_function: RewardFunction) -> RewardFunction:
        self.reward_funcs.append(reward_function)
        return reward_function

    def action_mask(self, observation: th.Tensor) -> th.Tensor:
        if self.action_codec is None:
            raise RuntimeError("continuous controls do not use a categorical action mask")
        return self.action_codec.mask(observation)

    def _custom_reward(self, actions, score_delta, done, terminated, truncated):
        if self._state is None or self._observation is None:
            raise RuntimeError("reset must be called before using custom rewards")
        context = RewardContext(
            current=self._carl_state(self._env.get_transition_state()),
            previous=self._state,
            current_observation=self._observation_of(self._env.get_obs()),
            previous_observation=self._observation,
            events=CarlEvents(score_delta=score_delta, done=done, terminated=terminated, truncated=truncated),
            actions=actions,
            score_difference=self._score_difference,
            episode_ticks=self._episode_ticks,
            overtime=self._overtime,
        )
        reward = th.zeros((self.n_sim, self.n_cars), device=self.device)
        info: dict[str, list[Any]] = {}
        for func in self.reward_funcs:
            result = func(context)
            if isinstance(result, RewardResult):
                info.update(result.info)
                result = result.reward
            if result.shape != reward.shape:
                raise ValueError(f"Reward must have shape {tuple(reward.shape)}")
            reward += result
        return (reward * self.reward_scale).reshape(self.n_envs), info

    # ------------------------------------------------------------ gym API

    def reset(self, *, seed: int | None = None, options: dict[str, Any] | None = None) -> th.Tensor:
        self._check_open()
        if seed is not None and seed != self._seed:
            raise ValueError("CARL's seed is constructor-only")
        if options:
            raise NotImplementedError("CARL reset options are not supported")
        self._sync()
        self._env.reset()
        self._apply_reset_state(th.ones(self.n_sim, dtype=th.bool, device=self.device))
        self._clear_sim_stats()
        return self._observe()

    def set_ball(self, position, velocity, angular_velocity, *, simulation_indices=None) -> th.Tensor:
        self._check_open()
        self._sync()
        self._env.set_ball(position.contiguous(), velocity.contiguous(), angular_velocity.contiguous(),
                           simulation_indices=(simulation_indices.contiguous()
                                               if simulation_indices is not None else None))
        return self._observe()

    def set_car(self, position, rotation, velocity, angular_velocity, demoed, *, boost=None, internal_state=None,
                simulation_indices=None) -> th.Tensor:
        self._check_open()
        self._sync()
        self._env.set_car(position.contiguous(), rotation.contiguous(), velocity.contiguous(),
                          angular_velocity.contiguous(), demoed.contiguous(),
                          boost=boost.contiguous() if boost is not None else None,
                          internal_state=internal_state.contiguous() if internal_state is not None else None,
                          simulation_indices=(simulation_indices.contiguous()
                                              if simulation_indices is not None else None))
        return self._observe()

    def step(self, actions):
        self._check_open()
        dtype = th.int32 if self.discrete_actions else th.float32
        actions = th.as_tensor(actions, dtype=dtype, device=self.device).contiguous()
        width = len(carl.ACTION_NVECS)
        if actions.shape != (self.n_envs, width):
            raise ValueError(f"Expected actions shaped {(self.n_envs, width)}")
        actions = actions.view(self.n_sim, self.n_cars, width)

        self._sync()
        if self.discrete_actions:
            self._env.step(actions)
        else:
            self._env.step_continuous(actions)
        self._sync()

        score_delta = self._tensor(self._env.get_rewards())
        sim_done = self._tensor(self._env.get_dones())
        self._score_difference = self._tensor(self._env.get_transition_score_difference())
        self._episode_ticks = self._tensor(self._env.get_transition_episode_ticks())
        self._overtime = self._tensor(self._env.get_transition_overtime())
        sim_terminated = sim_done & score_delta.ne(0)
        sim_truncated = sim_done & ~sim_terminated

        if self.reward_funcs:
            reward, reward_info = self._custom_reward(actions, score_delta, sim_done, sim_terminated, sim_truncated)
        else:
            reward = (score_delta[:, None] * self._team_sign).reshape(self.n_envs)
            reward_info = {}

        self._apply_reset_state(sim_done)
        self._clear_sim_stats(sim_done)
        obs = self._observe()

        terminated = self._per_car(sim_terminated)
        truncated = self._per_car(sim_truncated)
        done = terminated | truncated
        self._episode_return += reward
        self._episode_length += 1

        if self.defer_episode_reporting:
            self._episode_reports.append((self._episode_return.clone(), self._episode_length.clone(), done.clone()))
            self._episode_return.masked_fill_(done, 0)
            self._episode_length.masked_fill_(done, 0)
            info = {**reward_info, "final_obs": self._observation_of(self._env.get_transition_obs()),
                    "_final_obs": done}
            return obs, reward, terminated, truncated, info

        finished = done.nonzero(as_tuple=True)[0]
        info: dict[str, Any] = {"reward": [], "length": []}
        if finished.numel():
            info = {
                "reward": self._episode_return[finished].cpu().tolist(),
                "length": self._episode_length[finished].cpu().tolist(),
                "final_obs": self._observation_of(self._env.get_transition_obs()),
                "_final_obs": done,
                **reward_info,
            }
            self._episode_return[finished] = 0
            self._episode_length[finished] = 0
        return obs, reward, terminated, truncated, info

    def drain_episode_reports(self) -> dict[str, list[Any]]:
        """Completed episodes since the last drain, in step then actor order."""
        self._check_open()
        if not self._episode_reports:
            return {"reward": [], "length": []}
        returns, lengths, dones = zip(*self._episode_reports)
        finished = th.stack(dones).flatten().nonzero(as_tuple=True)[0]
        reports = {
            "reward": th.stack(returns).flatten()[finished].cpu().tolist(),
            "length": th.stack(lengths).flatten()[finished].cpu().tolist(),
        }
        self._episode_reports.clear()
        return reports

    def render(self) -> None:
        return None

    def close(self, **_: Any) -> None:
        if self.closed:
            return
        self._sync()
        del self._env
        self.closed = True


__all__ = ["CARLTorchVectorEnv", "ResetStateProvider", "RewardFunction"]
