"""Drop-in alias of carl_amd.gymnasium.torch."""
import sys as _sys

import carl_amd.gymnasium.torch as _impl

_sys.modules[__name__] = _impl
