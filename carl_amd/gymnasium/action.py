"""Categorical action codec with availability masks.

API-compatible with python/carl/gymnasium/action.py:8-38: the mask enables
powerslide only on the ground, boost only with boost left, and jump on the
ground or while the dodge window is still open for more than one tick.
"""
import torch as th
import torch.nn as nn

import carl_amd as carl
from carl_amd import ACTION_NVECS


class CARLActionCodec(nn.Module):
    def __init__(self, previous_controls: bool = False):
        super().__init__()
        self._controls_size = carl.OBS_PREVIOUS_CONTROLS if previous_controls else 0

    @property
    def action_shape(self) -> tuple[int, ...]:
        return (len(ACTION_NVECS),)

    def mask(self, observation: th.Tensor) -> th.Tensor:
        tail = self._controls_size
        on_ground = observation[..., carl.OBS_EGO_ON_GROUND_INDEX].bool()
        has_boost = observation[..., carl.OBS_EGO_BOOST_INDEX].gt(0)
        flip_open = observation[..., carl.OBS_EGO_FLIP_INDEX - tail].bool()
        window = observation[..., carl.OBS_EGO_DODGE_TIME_INDEX - tail]
        jump_ok = on_ground | (flip_open & (window > carl.PHYS_DT))

        mask = th.ones((*observation.shape[:-1], carl.ACTION_LOGITS), dtype=th.bool, device=observation.device)
        mask[..., carl.ACTION_POWERSLIDE_LOGIT] = on_ground
        mask[..., carl.ACTION_BOOST_LOGIT] = has_boost
        mask[..., carl.ACTION_JUMP_LOGIT] = jump_ok
        return mask


__all__ = ["ACTION_NVECS", "CARLActionCodec"]
