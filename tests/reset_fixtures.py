"""Shared inputs and guards for the reset-path tests.

The restored scene is the one the reference's reset tests use
(tests/test_resets.py:28-72): the ball 800 uu up moving along +x at
170 uu/s, the cars in a row 250 uu apart at y = -1000 resting on the floor,
unrotated, with 61 boost and the last car demolished, an internal state with
`has_jumped` and `last_jump` set, and a 2-1 score at tick 23.
"""
from __future__ import annotations

import torch
from torch.utils._python_dispatch import TorchDispatchMode

import carl
from carl.gymnasium.state import CARLBall, CARLCars, CARLMatchReset, CARLResetState

BALL = {"position": (0.0, 0.0, 800.0), "velocity": (170.0, 0.0, 0.0), "angular_velocity": (0.0, 0.0, 0.0)}
ROW_SPACING, ROW_X0, ROW_Y, REST_Z = 250.0, -500.0, -1000.0, 17.0
BOOST = 61.0
INTERNAL_SET = (3, 5)           # has_jumped, last_jump
SCORE, TICKS = (2, 1), 23


def reset_inputs(n_rows: int, n_cars: int, *, match: bool = True, internal: bool = True,
                 device: str | torch.device = "cpu") -> dict[str, torch.Tensor]:
    """Env.apply_reset_state keyword inputs for n_rows arenas."""
    def full(shape, value, dtype=torch.float32):
        return torch.full(shape, value, dtype=dtype, device=device)

    def filled(shape, row):
        # fresh contiguous storage (also for zero rows), every row = `row`
        t = full(shape, 0.0, row.dtype)
        t[...] = row
        return t

    out = {f"ball_{k}": filled((n_rows, 3), torch.tensor(v, device=device)) for k, v in BALL.items()}
    x = ROW_X0 + ROW_SPACING * torch.arange(n_cars, dtype=torch.float32, device=device)
    out["car_position"] = filled((n_rows, n_cars, 3),
                                 torch.stack((x, full((n_cars,), ROW_Y), full((n_cars,), REST_Z)), -1))
    out["car_rotation"] = filled((n_rows, n_cars, 4), torch.tensor((0.0, 0.0, 0.0, 1.0), device=device))
    out["car_velocity"] = full((n_rows, n_cars, 3), 0.0)
    out["car_angular_velocity"] = full((n_rows, n_cars, 3), 0.0)
    out["car_demoed"] = filled((n_rows, n_cars), torch.arange(n_cars, device=device) == n_cars - 1)
    out["car_boost"] = full((n_rows, n_cars), BOOST)
    if internal:
        state = full((n_rows, n_cars, carl.CAR_INTERNAL_SIZE), 0.0)
        state[..., list(INTERNAL_SET)] = 1.0
        out["car_internal_state"] = state
    if match:
        out["blue_score"] = full((n_rows,), SCORE[0], torch.int32)
        out["orange_score"] = full((n_rows,), SCORE[1], torch.int32)
        out["episode_ticks"] = full((n_rows,), TICKS, torch.int32)
    return out


def typed_reset_state(values: dict[str, torch.Tensor], indices: torch.Tensor | None = None, *,
                      reset_mask: torch.Tensor | None = None) -> CARLResetState:
    """The same restore as a CARLResetState (observation-layout car rows:
    unrotated cars have forward = +x and up = +z)."""
    pos = values["car_position"]
    rows, n_cars = pos.shape[:2]
    cars = CARLCars.from_tensor(pos.new_zeros(rows, n_cars, carl.OBS_PER_CAR), n_cars)
    cars.position.copy_(pos)
    cars.forward.copy_(pos.new_tensor((1.0, 0.0, 0.0)).expand_as(pos))
    cars.up.copy_(pos.new_tensor((0.0, 0.0, 1.0)).expand_as(pos))
    cars.boost.copy_(values["car_boost"])
    cars[..., carl.OBS_DEMOED] = values["car_demoed"].to(cars.dtype)
    ball = CARLBall.from_tensor(torch.cat([values[f"ball_{k}"] for k in BALL], dim=-1))
    match = CARLMatchReset(values["blue_score"], values["orange_score"], values["episode_ticks"])
    return CARLResetState(indices, ball, cars, values.get("car_internal_state"), match, reset_mask=reset_mask)


class NoHostSync(TorchDispatchMode):
    """Raises on every operator whose result size or value would have to come
    back to the host: scalar reads, nonzero, masked_select, unique and
    indexing with a boolean mask."""

    _BANNED = {
        torch.ops.aten._local_scalar_dense.default: "scalar read",
        torch.ops.aten.nonzero.default: "nonzero",
        torch.ops.aten.masked_select.default: "masked_select",
        torch.ops.aten._unique2.default: "unique",
    }

    def __torch_dispatch__(self, func, types, args=(), kwargs=None):
        why = self._BANNED.get(func)
        if why is None and func is torch.ops.aten.index.Tensor:
            if any(i is not None and i.dtype in (torch.bool, torch.uint8) for i in args[1]):
                why = "boolean-mask indexing"
        if why is not None:
            raise AssertionError(f"operation needs the host: {why}")
        return func(*args, **(kwargs or {}))
