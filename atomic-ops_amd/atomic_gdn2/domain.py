"""Domain of correctness of the operator and its guards (reference ``atomic_gdn2/domain.py``).

I-1: g <= 0.  I-2: beta * ||k||^2 <= 2.  I-3 (BTL diagonal): half_span < 88, where half_span is
the maximum over inner blocks of bs2 rows and channels of 0.5 * (gc[s0] - gc[s1-1]); past it one
BTL leg overflows float32 (0 * inf -> NaN -> 0 after sanitize), so it is checked by the maximum
and enforced by clamping g.  Same names, arguments and thresholds as the reference
(domain.py:14-62); torch tensors on any device instead of jax arrays.
"""
from __future__ import annotations

import math

import torch

from .config import BTL_HARD_LIMIT, BTL_STOP, BTL_WARN


def half_span_max(gc_chunks, bs2: int):
    """gc_chunks: (..., bt, D), the cumsum inside each chunk.  Max half span (0-d tensor)."""
    bt, D = gc_chunks.shape[-2:]
    blk = gc_chunks.reshape(gc_chunks.shape[:-2] + (bt // bs2, bs2, D))
    span = blk[..., 0, :] - blk[..., -1, :]
    return 0.5 * span.max()


def half_span_from_g(g_hm, bt: int, bs2: int):
    """g_hm: (B,H,L,D) -> max half span."""
    b, h, L, d = g_hm.shape
    gc = torch.cumsum(g_hm.float().reshape(b, h, L // bt, bt, d), dim=-2)
    return half_span_max(gc, bs2)


def bk2_stat(k, b):
    """(max, mean) of sum_d b * k^2 (I-2)."""
    x = (b * k * k).sum(-1)
    return x.max(), x.mean()


def clamp_g(g_neg, g_max: float):
    """g_neg <= 0; enforce |g| <= g_max (hard clamp; the gradient passes inside the range)."""
    return torch.clamp(g_neg, min=-g_max)


def init_g_bias(target: float = 0.05):
    """Bias so that softplus(bias) = target (slow forgetting at init)."""
    return math.log(math.expm1(target))


def check_preconditions(g_hm, cfg, strict=True):
    """Half-span status of a (B,H,L,D) gate: 'ok', 'warn' (> BTL_WARN) or 'STOP' (> BTL_STOP,
    raised as RuntimeError when strict).  Only the BTL diagonal has the limit."""
    hs = float(half_span_from_g(g_hm, cfg.bt, cfg.bs2)) if cfg.diag == "btl" else 0.0
    status = "ok"
    if hs > BTL_STOP:
        status = "STOP"
    elif hs > BTL_WARN:
        status = "warn"
    if strict and status == "STOP":
        raise RuntimeError(f"BTL half_span={hs:.1f} > {BTL_STOP} (limit {BTL_HARD_LIMIT}); reduce bs2 or clamp g")
    return {"half_span_max": hs, "status": status}


def safe_bs2_for(g_max: float, candidates=(128, 64, 32, 16, 8)):
    """Largest candidate bs2 whose worst-case half span g_max * bs2 / 2 stays below BTL_STOP."""
    for c in candidates:
        if g_max * c / 2.0 < BTL_STOP:
            return c
    return candidates[-1]
