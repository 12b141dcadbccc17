"""Gymnasium-style vector environment over the MI355X CARL engine."""
from .action import ACTION_NVECS, CARLActionCodec
from .state import (
    REGULATION_TICKS,
    CARLBall,
    CARLCar,
    CARLCars,
    CARLMatchReset,
    CARLObservation,
    CARLResetState,
    CarlEvents,
    CarlState,
    RewardContext,
    RewardResult,
)
from .torch import CARLTorchVectorEnv, ResetStateProvider, RewardFunction

__all__ = [
    "ACTION_NVECS",
    "CARLActionCodec",
    "CARLBall",
    "CARLCar",
    "CARLCars",
    "CARLMatchReset",
    "CARLObservation",
    "CARLResetState",
    "CARLTorchVectorEnv",
    "CarlEvents",
    "CarlState",
    "REGULATION_TICKS",
    "RewardContext",
    "RewardFunction",
    "RewardResult",
    "ResetStateProvider",
]
