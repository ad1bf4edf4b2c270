"""The chunk-parallel WY stage on the HIP kernels, exposed for stage-level checks.

``build_scores(q, k, b, gc, scale, cfg) -> (Aqk, Akk)`` is the reference's Kernel A entry
point (``fwd/scores.py:87-97``) with its signature: chunked (B,H,nc,bt,D) arrays (or
(B,H,L,D)), gc the caller's in-chunk cumulative gate, used as given (``gdn2_scores``).
``wy_stage(q, k, v, w, b, g, scale, cfg)`` runs the whole chunk-parallel stage from the raw
gate g (the in-chunk cumsum formed by the kernel, as the operator does) and also returns the
WY inverse and recompute of ``fwd/solve.py`` and ``fwd/cd_slim.py:12-21`` (``gdn2_wy_stage``).
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from .pipeline import _check_device, _f32


def wy_stage(q, k, v, w, b, g, scale, cfg):
    """q..g: (B,H,L,D) or chunked (B,H,nc,bt,D) on a ROCm device.  Returns a dict of chunked
    float32 tensors: aqk, akk, A (B,H,nc,bt,bt); wp, u, kg, qg (B,H,nc,bt,D); gl (B,H,nc,D)."""
    _check_device(q)
    if q.dim() == 5:
        B, H, nc, bt, D = q.shape
        q, k, v, w, b, g = (t.reshape(B, H, nc * bt, D) for t in (q, k, v, w, b, g))
    xs = [_f32(t) for t in (q, k, v, w, b, g)]
    B, H, L, D = xs[0].shape
    bt = cfg.bt
    if L % bt:
        raise ValueError(f"L={L} must be divisible by bt={bt}")
    nc = L // bt
    dev = xs[0].device
    mk = lambda *s: torch.empty(*s, dtype=torch.float32, device=dev)
    out = dict(aqk=mk(B, H, nc, bt, bt), akk=mk(B, H, nc, bt, bt), A=mk(B, H, nc, bt, bt),
               wp=mk(B, H, nc, bt, D), u=mk(B, H, nc, bt, D), kg=mk(B, H, nc, bt, D),
               qg=mk(B, H, nc, bt, D), gl=mk(B, H, nc, D))
    desc = _lib.make_desc(cfg, B, H, L, D, float(scale))
    with torch.cuda.device(dev):
        _lib.residual_layout(desc)                       # validates the descriptor
        _lib.check(_lib.lib().gdn2_wy_stage(ctypes.byref(desc), *map(_lib.ptr, xs),
                                            *(_lib.ptr(out[n]) for n in ("aqk", "akk", "A", "wp", "u", "kg", "qg", "gl")),
                                            _lib.stream_handle(dev)), "gdn2_wy_stage")
    return out


def build_scores(q, k, b, gc, scale, cfg):
    """(Aqk, Akk), masked and sanitized, chunked (B,H,nc,bt,bt) float32, from q, k, b and the
    in-chunk cumulative gate gc (fwd/scores.py:87-97)."""
    _check_device(q)
    if q.dim() == 5:
        B, H, nc, bt, D = q.shape
        q, k, b, gc = (t.reshape(B, H, nc * bt, D) for t in (q, k, b, gc))
    xs = [_f32(t) for t in (q, k, b, gc)]
    B, H, L, D = xs[0].shape
    bt = cfg.bt
    if L % bt:
        raise ValueError(f"L={L} must be divisible by bt={bt}")
    nc = L // bt
    dev = xs[0].device
    aqk = torch.empty(B, H, nc, bt, bt, dtype=torch.float32, device=dev)
    akk = torch.empty_like(aqk)
    desc = _lib.make_desc(cfg, B, H, L, D, float(scale))
    with torch.cuda.device(dev):
        _lib.residual_layout(desc)                       # validates the descriptor
        _lib.check(_lib.lib().gdn2_scores(ctypes.byref(desc), *map(_lib.ptr, xs), _lib.ptr(aqk), _lib.ptr(akk),
                                          _lib.stream_handle(dev)), "gdn2_scores")
    return aqk, akk
