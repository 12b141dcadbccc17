"""Categorical action codec with availability masks.

Interface and rules: python/carl/gymnasium/action.py:8-38.  Every logit of
the seven heads (ACTION_NVECS) is available except three, each tied to one
predicate of the observer's own observation: powerslide needs three wheels
on the ground, boost needs boost left, and jump needs the ground or an open
dodge window with more than one tick left in it.

The mask is a gather: each logit carries the index of its predicate in a
small table (0: always available), and the predicates of a batch of
observations are stacked once and indexed by that table.
"""
import torch as th
import torch.nn as nn

import carl_amd as carl
from carl_amd import ACTION_NVECS

_ALWAYS, _ON_GROUND, _HAS_BOOST, _CAN_JUMP = range(4)


class CARLActionCodec(nn.Module):
    def __init__(self, previous_controls: bool = False):
        super().__init__()
        # the dodge columns are counted from the end of the row, before the
        # optional previous controls
        self._tail = carl.OBS_PREVIOUS_CONTROLS if previous_controls else 0
        rule = th.full((carl.ACTION_LOGITS,), _ALWAYS, dtype=th.long)
        rule[carl.ACTION_POWERSLIDE_LOGIT] = _ON_GROUND
        rule[carl.ACTION_BOOST_LOGIT] = _HAS_BOOST
        rule[carl.ACTION_JUMP_LOGIT] = _CAN_JUMP
        self.register_buffer("_rule", rule, persistent=False)

    @property
    def action_shape(self) -> tuple[int, ...]:
        return (len(ACTION_NVECS),)

    def mask(self, observation: th.Tensor) -> th.Tensor:
        on_ground = observation[..., carl.OBS_EGO_ON_GROUND_INDEX] != 0
        has_boost = observation[..., carl.OBS_EGO_BOOST_INDEX] > 0
        dodge_open = observation[..., carl.OBS_EGO_FLIP_INDEX - self._tail] != 0
        window = observation[..., carl.OBS_EGO_DODGE_TIME_INDEX - self._tail]
        can_jump = on_ground | (dodge_open & (window > carl.PHYS_DT))
        predicates = th.stack((th.ones_like(on_ground), on_ground, has_boost, can_jump), dim=-1)
        return predicates[..., self._rule.to(observation.device)]


__all__ = ["ACTION_NVECS", "CARLActionCodec"]
