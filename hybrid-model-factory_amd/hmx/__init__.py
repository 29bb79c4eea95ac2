"""hmx — MI355X (gfx950) linear-recurrent mixer ops behind the reference's Python signatures.

Host side: PyTorch-ROCm for device memory and streams; compute: hand-written
HIP kernels in libhmx.so reached through the C ABI in include/hmx.h.
"""
from . import _lib
from .ops import *  # noqa: F401,F403
from .ops import __all__ as _ops_all

__all__ = list(_ops_all)
__version__ = "0.1.0"
