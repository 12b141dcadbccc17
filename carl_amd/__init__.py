"""carl_amd - CARL step engine for AMD Instinct MI355X.

Drop-in for the reference `carl` package: `carl_amd.Env` is the native
environment (HIP kernels behind the C-ABI in include/carl_amd.h) and every
upper-case module constant of the reference binding is re-exported.
"""
import os
from pathlib import Path

_arena = Path(__file__).with_name("assets") / "arena.obj"
os.environ.setdefault("CARL_ARENA_OBJ", str(_arena))

import torch as _torch  # noqa: E402  (DLPack consumer; loaded before the extension)

try:
    from . import _carl  # noqa: E402
except ImportError as exc:  # the product has no CPU fallback
    raise ImportError(
        "carl_amd requires its native HIP extension (libcarl_amd.so and _carl); "
        "build it with `python carl_amd/build.py` "
        f"(PyTorch {_torch.__version__})"
    ) from exc

__all__ = [name for name in vars(_carl) if name == "Env" or name.isupper()]
globals().update({name: getattr(_carl, name) for name in __all__})
