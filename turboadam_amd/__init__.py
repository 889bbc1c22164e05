"""turboadam_amd -- MI355X-native TurboAdam (fused packed-state optimizer step).

Drop-in for davidkny22/turboadam's `TurboAdam` (src/turboadam/__init__.py).
"""

from importlib.metadata import PackageNotFoundError, version

try:
    __version__ = version("turboadam_amd")
except PackageNotFoundError:
    __version__ = "0.1.0"

from .checkpoint import load_reference_checkpoint  # noqa: E402
from .optimizer import TurboAdam  # noqa: E402

__all__ = ["TurboAdam", "load_reference_checkpoint"]
