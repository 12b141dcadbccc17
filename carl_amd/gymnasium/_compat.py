"""Gymnasium types, or minimal stand-ins when gymnasium is not installed.

The vector environment only needs Box / MultiDiscrete spaces (shape, dtype,
bounds), batch_space and the VectorEnv base with the SAME_STEP autoreset mode.
"""
from __future__ import annotations

import enum

import numpy as np

try:  # pragma: no cover - exercised only where gymnasium exists
    import gymnasium as _gym
    from gymnasium.vector import AutoresetMode, VectorEnv
    from gymnasium.vector.utils import batch_space

    Box = _gym.spaces.Box
    MultiDiscrete = _gym.spaces.MultiDiscrete
    HAVE_GYMNASIUM = True
except ImportError:
    HAVE_GYMNASIUM = False

    class AutoresetMode(enum.Enum):
        NEXT_STEP = "NextStep"
        SAME_STEP = "SameStep"
        DISABLED = "Disabled"

    class VectorEnv:
        metadata: dict = {}
        closed = False

        def __init__(self) -> None:
            pass

    class Box:
        def __init__(self, low, high, shape=None, dtype=np.float32):
            self.dtype = np.dtype(dtype)
            if shape is None:
                shape = np.shape(low)
            self.shape = tuple(int(s) for s in shape)
            self.low = np.broadcast_to(np.asarray(low, dtype=self.dtype), self.shape).copy()
            self.high = np.broadcast_to(np.asarray(high, dtype=self.dtype), self.shape).copy()

        def __repr__(self) -> str:
            return f"Box({self.shape}, {self.dtype})"

    class MultiDiscrete:
        def __init__(self, nvec, dtype=np.int64):
            self.nvec = np.asarray(nvec, dtype=np.int64)
            self.dtype = np.dtype(dtype)
            self.shape = self.nvec.shape

        def __repr__(self) -> str:
            return f"MultiDiscrete({self.nvec.tolist()})"

    def batch_space(space, n: int):
        if isinstance(space, Box):
            return Box(np.stack([space.low] * n), np.stack([space.high] * n), (n, *space.shape), space.dtype)
        if isinstance(space, MultiDiscrete):
            return MultiDiscrete(np.stack([space.nvec] * n), space.dtype)
        raise TypeError(f"cannot batch {space!r}")
