"""Runtime canary: BTL scores against exact (lean) scores on a sample of chunks (reference
``atomic_gdn2/training/canary.py:12-23``).  Both score sets come from the HIP kernels
(``build_scores`` with ``diag='btl'`` and ``diag='lean'`` on the same gc); the alarm fires when their Akk
differ by more than ``thresh`` in relative L2, which flags a gate whose half span has left the
BTL factorisation's domain."""
from __future__ import annotations

import numpy as np
import torch

from ..domain import half_span_max
from ..stages import build_scores


def _rel(a, b):
    a, b = a.double(), b.double()
    return float((a - b).norm() / max(float(b.norm()), 1e-12))


def btl_vs_lean_canary(cfg, q=None, k=None, b=None, g=None, D=64, g_level=None, thresh=1e-3, seed=0,
                       device="cuda"):
    """q, k, b, g: (B,H,nc,bt,D) chunks (a sample).  If omitted: one synthetic chunk with
    constant |g| = g_level."""
    if q is None:
        rng = np.random.default_rng(seed)
        sh = (1, 1, 1, cfg.bt, D)
        q, k = (torch.from_numpy(rng.normal(size=sh).astype(np.float32) * 0.3).to(device) for _ in range(2))
        b = torch.from_numpy(np.abs(rng.normal(size=sh)).astype(np.float32) * 0.5).to(device)
        g = torch.full(sh, -float(g_level), dtype=torch.float32, device=device)
    gc = torch.cumsum(g.float(), dim=-2)
    scale = 1.0 / np.sqrt(q.shape[-1])
    _, Ab = build_scores(q, k, b, gc, scale, cfg.with_(diag="btl"))
    _, Al = build_scores(q, k, b, gc, scale, cfg.with_(diag="lean"))
    err = _rel(Ab, Al)
    return dict(rel_err=err, half_span=float(half_span_max(gc, cfg.bs2)), alarm=err > thresh)
