"""Legacy kernel configuration, sanitize helpers and input validation (reference
``atomic_ops/configs.py:16-52`` and ``116-136``): same fields, presets, checks and messages."""
from __future__ import annotations

import dataclasses as dc

import torch


@dc.dataclass(frozen=True)
class KernelConfig:
    bt: int = 256
    bc: int = 128
    mb: int = 16
    clip: float = 1e4
    wy_eps: float = 0.0

    @property
    def n_sub(self) -> int:
        return self.bt // self.bc

    @property
    def n_micro(self) -> int:
        return self.bc // self.mb

    def __post_init__(self):
        if self.bt % self.bc != 0:
            raise ValueError(f"bt={self.bt} must be divisible by bc={self.bc}")
        if self.bt != 2 * self.bc:
            raise ValueError(f"bt={self.bt} must equal 2*bc (top-level WY-solve split supports only "
                             f"the 2-block case); got bc={self.bc}. Vary `mb` instead of `bc`.")
        if self.bc % self.mb != 0:
            raise ValueError(f"bc={self.bc} must be divisible by mb={self.mb}")
        if not (0.0 <= self.wy_eps < 1.0):
            raise ValueError(f"wy_eps={self.wy_eps} must be in [0, 1)")


KAGGLE_SMALL = KernelConfig(bt=128, bc=64, mb=16, clip=1e4, wy_eps=1e-3)
KAGGLE_MEDIUM = KernelConfig(bt=256, bc=128, mb=16, clip=1e4, wy_eps=1e-3)
KAGGLE_LARGE = KernelConfig(bt=256, bc=128, mb=16, clip=5e3, wy_eps=1e-3)
DEFAULT_CONFIG = KAGGLE_MEDIUM


def sanitize(x, config: KernelConfig = DEFAULT_CONFIG):
    """clip to +-clip, NaN -> 0, +-inf -> +-clip."""
    c = config.clip
    return torch.nan_to_num(torch.clamp(x, -c, c), nan=0.0, posinf=c, neginf=-c)


def sanitize_h0(h0, config: KernelConfig = DEFAULT_CONFIG):
    return sanitize(h0, config)


def clip_acc(x, config: KernelConfig = DEFAULT_CONFIG):
    return sanitize(x, config)


def validate_inputs(q, k, v, w, b, g, scale, h0, config: KernelConfig):
    """Shape checks of the legacy entry points; returns (bsz, L, H, D, n_chunks)."""
    if q.ndim != 4:
        raise ValueError(f"q must be (batch, seq_len, heads, d_head); got shape {tuple(q.shape)}")
    bsz, L, H, D = q.shape
    if D != 128:
        raise ValueError(f"Kernels assume d_head=128 (MXU tile); got D={D}.")
    if L % config.bt != 0:
        raise ValueError(f"seq_len={L} must be divisible by config.bt={config.bt}.")
    for name, t in (("k", k), ("v", v), ("w", w), ("b", b), ("g", g)):
        if tuple(t.shape) != tuple(q.shape):
            raise ValueError(f"{name}.shape={tuple(t.shape)} must match q.shape={tuple(q.shape)}")
    if h0 is not None and tuple(h0.shape) != (bsz, H, D, D):
        raise ValueError(f"h0.shape={tuple(h0.shape)} must be {(bsz, H, D, D)}")
    return bsz, L, H, D, L // config.bt
