"""Legacy entry points (reference ``atomic_ops/fallback.py:9-22``,
``gdn2_fwd.py:340-361``, ``gdn2_pipeline.py:145-152``) over the GDN-2 operator.

Inputs are (batch, seq_len, heads, d_head) with d_head = 128; ``config`` is a legacy
``KernelConfig`` (chunk ``bt``, leaf ``mb``, ``clip``, ``wy_eps``).  Returns
(o (batch, seq_len, heads, d_head) float32, h_final (batch, heads, d_head, d_head) float32).

Which operator runs.  The reference dispatches on the device (fallback.py:9-22): its Pallas
path runs chunk ``config.bt`` with ``config.wy_eps``; everywhere else it runs
``gdn2_chunked_wy_reference(..., chunk_size=config.bt)`` with that function's default
``wy_eps = 0`` (reference.py:109).  The (1 - wy_eps) damping acts on the coupling inside a
chunk only, so with wy_eps > 0 the chunk size is part of the operator; with wy_eps = 0 the
chunked WY form equals the token recurrence for every chunk size and only the rounding
depends on it.  This shim therefore runs chunk ``config.bt`` with ``config.wy_eps`` when the
HIP kernels run that chunk (64, 128 and 256: every preset, as the reference's TPU path runs
them), and otherwise the reference's off-TPU operator: wy_eps = 0, at the kernels' chunk of
64.  Products are fp32
everywhere (the legacy kernels use Precision.HIGHEST).
"""
from __future__ import annotations


from atomic_gdn2 import make_cfg, make_blr_trainable
from atomic_gdn2.pipeline import kernels_support

from .configs import DEFAULT_CONFIG, KernelConfig, validate_inputs

_OPS = {}


def _operator(config: KernelConfig, scale: float):
    key = (config, float(scale))
    fn = _OPS.get(key)
    if fn is None:
        fn = _OPS[key] = make_blr_trainable(operator_cfg(config), scale)
    return fn


def operator_cfg(config: KernelConfig):
    """The operator configuration that stands in for ``config`` (see the module docstring).

    Scores: the legacy Kernel A forms every score pair exactly, exp(clip(gc_i - gc_j, -20, 20))
    per channel over the whole chunk (atomic_ops/gdn2_fwd.py:60-65, and the same in its off-TPU
    reference, reference.py:73-74), so the operator runs the exact ('lean') diagonal with
    diff_clip 20 on the largest diagonal block the kernels take: bs2 = 64.  At bt = 64 that is
    the whole chunk, as in the legacy kernel; at bt = 128 / 256 the pairs in different 64-token
    parts are carried by the state, exactly and without the clip (the two differ only where
    gc_i - gc_j < -20 across parts, i.e. for pair weights below e^-20)."""
    bt = config.bt if kernels_support(config.bt, config.wy_eps) else 64
    eps = config.wy_eps if bt == config.bt else 0.0
    return make_cfg(bt=bt, bc=bt // 2, score_bs=bt, bs2=64, mb=min(config.mb, bt),
                    diag="lean", diff_clip=20.0, clip=config.clip, wy_eps=eps, dot_mode="highest",
                    solve_dot_mode="highest", b3_dot_mode="highest")


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
