"""Legacy entry points (reference ``atomic_ops/fallback.py:9-22``,
``gdn2_fwd.py:340-361``, ``gdn2_pipeline.py:145-152``) over the GDN-2 operator.

Inputs are (batch, seq_len, heads, d_head) with d_head = 128; ``config`` is a legacy
``KernelConfig`` whose chunk size ``bt`` the legacy validation still requires to divide seq_len.
The operator itself always runs at this build's chunk of 64 tokens (the chunked WY form is exact
for any chunk size; only rounding differs), with the legacy ``clip``, ``wy_eps`` and leaf size
``mb`` and fp32 products everywhere (the legacy kernels use Precision.HIGHEST).  Returns
(o (batch, seq_len, heads, d_head) float32, h_final (batch, heads, d_head, d_head) float32).
"""
from __future__ import annotations


from atomic_gdn2 import make_cfg, make_blr_trainable

from .configs import DEFAULT_CONFIG, KernelConfig, validate_inputs

_OPS = {}


def _operator(config: KernelConfig, scale: float):
    key = (config, float(scale))
    fn = _OPS.get(key)
    if fn is None:
        mb = min(config.mb, 64)
        cfg = make_cfg(bt=64, bc=32, score_bs=64, bs2=32, mb=mb, diag="btl", clip=config.clip,
                       wy_eps=config.wy_eps, dot_mode="highest", solve_dot_mode="highest",
                       b3_dot_mode="highest")
        fn = _OPS[key] = make_blr_trainable(cfg, scale)
    return fn


def _run(q, k, v, w, b, g, scale, h0, config):
    config = config or DEFAULT_CONFIG
    validate_inputs(q, k, v, w, b, g, scale, h0, config)
    sw = lambda x: x.transpose(1, 2)
    o, hf = _operator(config, scale)(*(sw(x) for x in (q, k, v, w, b, g)), h0)
    return sw(o), hf


def gdn2_forward(q, k, v, w, b, g, scale, h0=None, config=None):
    return _run(q, k, v, w, b, g, scale, h0, config)


def gdn2_forward_trainable(q, k, v, w, b, g, scale, h0=None, config=None):
    return _run(q, k, v, w, b, g, scale, h0, config)


def gdn2_pallas_forward(q, k, v, w, b, g, scale, h0=None, config: KernelConfig = DEFAULT_CONFIG, debug_tag: str = ""):
    return _run(q, k, v, w, b, g, scale, h0, config)


def gdn2_pallas_forward_trainable(q, k, v, w, b, g, scale, h0=None, config: KernelConfig = DEFAULT_CONFIG):
    return _run(q, k, v, w, b, g, scale, h0, config)
