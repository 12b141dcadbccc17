"""Drop-in alias of carl_amd.gymnasium.action."""
import sys as _sys

import carl_amd.gymnasium.action as _impl

_sys.modules[__name__] = _impl
