"""Drop-in alias of carl_amd.gymnasium."""
from carl_amd.gymnasium import *  # noqa: F401,F403
from carl_amd.gymnasium import __all__  # noqa: F401
