"""Drop-in alias of carl_amd.gymnasium.state."""
import sys as _sys

import carl_amd.gymnasium.state as _impl

_sys.modules[__name__] = _impl
