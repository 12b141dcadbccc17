"""Drop-in import name: `import carl` resolves to the carl_amd engine."""
import carl_amd as _impl
from carl_amd import *  # noqa: F401,F403

__all__ = list(_impl.__all__)
_carl = _impl._carl
