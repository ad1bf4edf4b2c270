"""atomic_ops -- the reference's legacy API (``atomic_ops/__init__.py``) as a thin layer over
the GDN-2 operator on the MI355X HIP kernels (``atomic_gdn2``).

Legacy callers keep their (batch, seq_len, heads, d_head) layout, ``KernelConfig`` presets and
entry points; every call transposes to head-major and runs ``atomic_gdn2.make_blr_trainable``
(no dual dispatch: there is no CPU or reference fallback).  The legacy package's JAX reference
implementations (``gdn2_chunked_wy_reference``, ``gdn2_token_serial_reference``) are test
oracles and are not part of this layer.
"""
from .configs import KernelConfig, KAGGLE_SMALL, KAGGLE_MEDIUM, KAGGLE_LARGE, DEFAULT_CONFIG
from .utils import is_tpu_available, is_hip_available, estimate_memory, get_recommended_config
from .fallback import gdn2_forward, gdn2_forward_trainable, gdn2_pallas_forward, gdn2_pallas_forward_trainable

__version__ = "0.2.0"

__all__ = [
    "KernelConfig", "KAGGLE_SMALL", "KAGGLE_MEDIUM", "KAGGLE_LARGE", "DEFAULT_CONFIG",
    "is_tpu_available", "is_hip_available", "estimate_memory", "get_recommended_config",
    "gdn2_forward", "gdn2_forward_trainable", "gdn2_pallas_forward", "gdn2_pallas_forward_trainable",
]
