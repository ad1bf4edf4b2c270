"""Seeded synthetic inputs for benchmarks and tests.

Recipe: ``numpy.random.Generator(PCG64(seed))`` draws ``standard_normal((B,H,L,D))`` in float64
in the fixed order q, k, v, w, b, g; then q, k and w are L2-normalised over D, v is kept,
``b = sigmoid(N)``, ``g = -0.1 * softplus(N)``; everything is cast to float32.  The scale is
``1/sqrt(D)`` and h0 = 0.  This is the benchmark distribution of the operator's gradient
workload (q,k L2-normalised rows, gates in (0,1), negative log-decays).
"""
from __future__ import annotations

import hashlib

import numpy as np


def make_inputs_np(B: int, H: int, L: int, D: int, seed: int = 0):
    """Returns (q, k, v, w, b, g) float32 arrays of shape (B,H,L,D) and the scale."""
    rng = np.random.Generator(np.random.PCG64(seed))
    sh = (B, H, L, D)
    q, k, v, w, b, g = (rng.standard_normal(sh) for _ in range(6))
    l2 = lambda x: x / np.linalg.norm(x, axis=-1, keepdims=True)
    q, k, w = l2(q), l2(k), l2(w)
    b = 1.0 / (1.0 + np.exp(-b))
    g = -0.1 * np.logaddexp(0.0, g)
    out = tuple(np.ascontiguousarray(x.astype(np.float32)) for x in (q, k, v, w, b, g))
    return out, 1.0 / np.sqrt(D)


def inputs_sha256(arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def make_inputs(B: int, H: int, L: int, D: int, seed: int = 0, device="cuda", dtype=None):
    """torch tensors on ``device`` (float32, or ``dtype``) and the scale."""
    import torch
    arrs, scale = make_inputs_np(B, H, L, D, seed)
    ts = tuple(torch.from_numpy(a).to(device) for a in arrs)
    if dtype is not None:
        ts = tuple(t.to(dtype) for t in ts)
    return ts, scale


def make_inputs_device(B: int, H: int, L: int, D: int, seed: int = 0, device="cuda", dtype=None):
    """The same distributions drawn by torch's generator on ``device`` (for workloads too large
    to draw on the host, e.g. the long-context forward): q, k, w L2-normalised rows, v ~ N(0,1),
    b = sigmoid(N), g = -0.1 softplus(N); float32, cast to ``dtype`` if given."""
    import torch
    gen = torch.Generator(device=device).manual_seed(seed)
    sh = (B, H, L, D)
    q, k, v, w, b, g = (torch.randn(sh, generator=gen, device=device) for _ in range(6))
    l2 = lambda x: x / torch.linalg.vector_norm(x, dim=-1, keepdim=True)
    q, k, w = l2(q), l2(k), l2(w)
    b = torch.sigmoid(b)
    g = -0.1 * torch.nn.functional.softplus(g)
    ts = (q, k, v, w, b, g)
    if dtype is not None:
        ts = tuple(t.to(dtype) for t in ts)
    return ts, 1.0 / D ** 0.5
