"""Legacy utilities (reference ``atomic_ops/utils.py``): device probe, memory estimate, preset
choice (same formula and thresholds)."""
from __future__ import annotations

from .configs import KernelConfig, KAGGLE_SMALL, KAGGLE_MEDIUM, KAGGLE_LARGE


def is_tpu_available() -> bool:
    """Kept for drop-in imports: this build runs on MI355X, never on a TPU."""
    return False


def is_hip_available() -> bool:
    try:
        import torch
        return bool(torch.cuda.is_available() and torch.version.hip)
    except Exception:
        return False


def estimate_memory(batch: int, seq_len: int, heads: int, d_head: int = 128, bt: int = 256,
                    bytes_per_param: int = 4) -> float:
    """Rough per-device residual memory in MB of the legacy chunked forward."""
    n_chunks = seq_len // bt
    per_chunk = (bt * bt * 3) + (bt * d_head * 7) + (d_head * d_head * 2)
    return batch * heads * n_chunks * per_chunk * bytes_per_param / (1024 * 1024)


def get_recommended_config(batch: int, seq_len: int, heads: int, d_head: int = 128) -> KernelConfig:
    mem = estimate_memory(batch, seq_len, heads, d_head)
    if mem > 6000:
        return KAGGLE_LARGE
    if mem > 2500:
        return KAGGLE_MEDIUM
    return KAGGLE_SMALL
