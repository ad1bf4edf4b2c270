"""atomic_gdn2 -- Gated DeltaNet-2 operator on MI355X (gfx950) HIP kernels.

Drop-in for the reference package's public API (reference atomic_gdn2/__init__.py:4-5):
``make_cfg``, ``BLRConfig``, ``PROD``, ``make_blr_trainable``.
"""
from .config import BLRConfig, make_cfg, PROD
from .pipeline import make_blr_trainable

__version__ = "0.2.0"

__all__ = ["BLRConfig", "make_cfg", "PROD", "make_blr_trainable", "__version__"]
