"""The operator: ``make_blr_trainable(cfg, scale)(q, k, v, w, b, g, h0=None) -> (o, h_final)``.

Drop-in for the reference's ``atomic_gdn2/pipeline.py:17-66``:

* head-major ``(B,H,L,D)`` inputs of any float dtype, ``L % cfg.bt == 0`` (else ValueError);
* ``o`` (B,H,L,D) and ``h_final`` (B,H,D,D) are float32 whatever the input dtype;
* sequences longer than ``cfg.max_chunks_per_call`` chunks are split into segments with the
  state carried through ``h0``/``h_final`` (pipeline.py:57-64);
* the call is one custom autograd node (the analogue of the reference's per-segment
  ``jax.custom_vjp``): its forward runs the HIP forward (``gdn2_fwd``) segment by segment and
  keeps each segment's residual buffer, its backward runs ``gdn2_bwd`` over the segments in
  reverse and returns each segment's gradients through ``_fin`` (pipeline.py:11-14): sanitized
  at 1e4 and cast back to each input's dtype.  Segments are views into the full tensors
  (``gdn2_desc.seq_ld``): no slice copies, gradient scatters or concatenation.

Every call goes to the HIP kernels in ``libgdn2_hip.so``; there is no other backend.  Tensors
must live on a ROCm device.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from .precision import sanitize

_FINAL_CLIP = 1e4
# chunk sizes (cfg.bt) the HIP kernels run (bt = 128 / 256 as 2 / 4 parts of 64 tokens, exactly)
SUPPORTED_BT = (64, 128, 256)


def kernels_support(bt, wy_eps):
    """Whether the HIP kernels run chunk ``bt`` with damping ``wy_eps``."""
    return bt in SUPPORTED_BT and 0.0 <= wy_eps < 1.0


# How the residual keeps the state for the backward (gdn2_desc.state_ckpt): K >= 1 keeps the
# state entering the first chunk of each checkpoint block (blocks of K chunks; up to two chunks
# left over become blocks of their own) and the backward recomputes the others inside its state
# reductions; 0 keeps every chunk's (as the reference's residual does, pipeline.py:25).
# K = 3 keeps 12 of every 32 states at or slightly below the stored form's time (MI355X, B4 H6
# D128, rounds interleaved: 0.5024 vs 0.5043 ms at L = 2048, 0.9726 vs 0.9776 ms at L = 4096);
# K = 4 keeps a quarter for 2 % more time, K = 8 an eighth for 8 %.
DEFAULT_STATE_CKPT = 3


def _fin(x, dt, cfg):
    """pipeline.py:11-14: pass through if already in dtype and clipped at <= 1e4."""
    if x.dtype == dt and cfg.clip <= _FINAL_CLIP:
        return x
    return sanitize(x, _FINAL_CLIP).to(dt)


def _f32(t):
    return t.to(torch.float32).contiguous()


def _check_inputs(ts, names):
    q = ts[0]
    if q.dim() != 4:
        raise ValueError(f"expected (B,H,L,D) inputs, got q.shape={tuple(q.shape)}")
    if q.numel() == 0:
        # the reference's segment loop has nothing to concatenate at L = 0 and fails there
        # (pipeline.py:57-64); the kernels need at least one chunk of one sequence
        raise ValueError(f"empty input q.shape={tuple(q.shape)}: B, H, L and D must be positive")
    for t, n in zip(ts, names):
        if t.shape != q.shape:
            raise ValueError(f"{n}.shape={tuple(t.shape)} differs from q.shape={tuple(q.shape)}")
        if not t.is_floating_point():
            raise TypeError(f"{n} must be a floating-point tensor")
        if t.device != q.device:
            raise ValueError(f"{n} is on {t.device}, q on {q.device}")


def _check_device(q):
    if q.device.type != "cuda":
        raise RuntimeError("atomic_gdn2 runs on the HIP kernels only: move the inputs to a ROCm "
                           f"device (got {q.device})")


def _segments(L, cfg):
    """Token ranges of the reference's segment loop: at most max_chunks_per_call chunks each
    (pipeline.py:57-64)."""
    step = cfg.max_chunks_per_call * cfg.bt
    return [(t0, min(L, t0 + step)) for t0 in range(0, L, step)]


def make_blr_trainable(cfg, scale, state_ckpt=None):
    """``state_ckpt``: this build's residual knob (no counterpart in the reference), see
    DEFAULT_STATE_CKPT; it changes memory and time, not results (the recomputed states equal
    the stored ones bit for bit)."""
    scale = float(scale)
    ckpt = DEFAULT_STATE_CKPT if state_ckpt is None else int(state_ckpt)
    if ckpt < 0:
        raise ValueError(f"state_ckpt={ckpt} must be >= 0")

    class _Sequence(torch.autograd.Function):
        """The whole call as one autograd node.  Forward and backward run the reference's
        segment loop (pipeline.py:57-64) over views of the full tensors: each segment's kernels
        read its inputs and write its o and gradients in place (gdn2_desc.seq_ld), the state
        is carried through h0 / h_final forward and through dh0 / dh_final backward, and each
        segment's gradients pass through ``_fin`` as the reference's per-segment custom_vjp
        returns them (so the dh handed to the previous segment is _fin(dh0, float32))."""

        @staticmethod
        def forward(ctx, q, k, v, w, b, g, h0):
            # h0 None = zero initial state (the kernel takes a null pointer; no zero fill)
            dts = tuple(t.dtype for t in (q, k, v, w, b, g)) + ((h0.dtype,) if h0 is not None else (torch.float32,))
            xs = [_f32(t) for t in (q, k, v, w, b, g)]
            h = None if h0 is None else _f32(h0)
            B, H, L, D = xs[0].shape
            dev = xs[0].device
            need_res = any(ctx.needs_input_grad)
            o = torch.empty((B, H, L, D), dtype=torch.float32, device=dev)
            L_ = _lib.lib()
            segs, res_list = [], []
            with torch.cuda.device(dev):
                stream = _lib.stream_handle(dev)
                for t0, t1 in _segments(L, cfg):
                    desc = _lib.make_desc(cfg, B, H, t1 - t0, D, scale, seq_ld=L, state_ckpt=ckpt)
                    _, tot = _lib.residual_layout(desc)      # validates the descriptor
                    res = torch.empty(tot, dtype=torch.uint8, device=dev) if need_res else None
                    ws = torch.empty(L_.gdn2_fwd_workspace_bytes(ctypes.byref(desc), int(need_res)),
                                     dtype=torch.uint8, device=dev)
                    hf = torch.empty((B, H, D, D), dtype=torch.float32, device=dev)
                    off = t0 * D
                    _lib.check(L_.gdn2_fwd(ctypes.byref(desc), *(_lib.ptr(x, off) for x in xs), _lib.ptr(h),
                                           _lib.ptr(o, off), _lib.ptr(hf), _lib.ptr(res), _lib.ptr(ws), stream),
                               "gdn2_fwd")
                    segs.append((t0, desc))
                    res_list.append(res)
                    h = hf
            if need_res:
                ctx.save_for_backward(*xs, *res_list)
                ctx.segs = segs
                ctx.dts = dts
            return o, h

        @staticmethod
        def backward(ctx, do, dhf):
            saved = ctx.saved_tensors
            xs, res_list = saved[:6], saved[6:]
            q = xs[0]
            B, H, L, D = q.shape
            dev = q.device
            do = torch.zeros_like(q) if do is None else _f32(do)
            dh = q.new_zeros((B, H, D, D)) if dhf is None else _f32(dhf)
            grads = [torch.empty_like(q) for _ in range(6)]
            L_ = _lib.lib()
            with torch.cuda.device(dev):
                stream = _lib.stream_handle(dev)
                for (t0, desc), res in reversed(list(zip(ctx.segs, res_list))):
                    ws = torch.empty(L_.gdn2_bwd_workspace_bytes(ctypes.byref(desc)), dtype=torch.uint8, device=dev)
                    dh0 = q.new_empty((B, H, D, D))
                    off = t0 * D
                    _lib.check(L_.gdn2_bwd(ctypes.byref(desc), *(_lib.ptr(x, off) for x in xs), _lib.ptr(res),
                                           _lib.ptr(do, off), _lib.ptr(dh), *(_lib.ptr(x, off) for x in grads),
                                           _lib.ptr(dh0), _lib.ptr(ws), stream), "gdn2_bwd")
                    # cotangent of the previous segment's h_final (float32), or of the caller's h0
                    dh = dh0 if t0 == 0 else _fin(dh0, torch.float32, cfg)
            out = tuple(_fin(x, dt, cfg) for x, dt in zip(grads, ctx.dts[:6]))
            return out + ((_fin(dh, ctx.dts[6], cfg),) if ctx.needs_input_grad[6] else (None,))

    def forward_only(xs, h0):
        """No gradient needed: one kernel sequence over all L (no residual kept).  Equal bit for
        bit to the segment loop, whose segments only bound the residual memory: the scan
        carries the fp32 state across chunk boundaries exactly as through h0 / h_final.  bf16
        inputs go to the kernels as they are (widened on load); other dtypes are cast to fp32."""
        q = xs[0]
        B, H, L, D = q.shape
        dev = q.device
        bf16 = all(t.dtype == torch.bfloat16 for t in xs)
        xs = [t.contiguous() if bf16 else _f32(t) for t in xs]
        h0c = None if h0 is None else _f32(h0)
        desc = _lib.make_desc(cfg, B, H, L, D, scale)
        o = torch.empty((B, H, L, D), dtype=torch.float32, device=dev)
        hf = torch.empty((B, H, D, D), dtype=torch.float32, device=dev)
        L_ = _lib.lib()
        with torch.cuda.device(dev):
            # (an invalid descriptor gives 0 bytes here and a ValueError from the call below)
            ws = torch.empty(L_.gdn2_fwd_workspace_bytes(ctypes.byref(desc), 0), dtype=torch.uint8, device=dev)
            entry = L_.gdn2_fwd_bf16 if bf16 else L_.gdn2_fwd
            _lib.check(entry(ctypes.byref(desc), *map(_lib.ptr, xs), _lib.ptr(h0c), _lib.ptr(o), _lib.ptr(hf),
                             None, _lib.ptr(ws), _lib.stream_handle(dev)),
                       "gdn2_fwd_bf16" if bf16 else "gdn2_fwd")
        return o, hf

    def call(q, k, v, w, b, g, h0=None):
        """q..g: (B,H,L,D), L % bt == 0. Returns (o (B,H,L,D) f32, h_final (B,H,D,D) f32)."""
        _check_inputs((q, k, v, w, b, g), "qkvwbg")
        bsz, H, L, D = q.shape
        if L % cfg.bt:
            raise ValueError(f"L={L} must be divisible by bt={cfg.bt}")
        h = h0
        if h is not None and h.shape != (bsz, H, D, D):
            raise ValueError(f"h0.shape={tuple(h.shape)} must be {(bsz, H, D, D)}")
        _check_device(q)
        xs = (q, k, v, w, b, g)
        if not (torch.is_grad_enabled() and any(t.requires_grad for t in xs + ((h,) if h is not None else ()))):
            return forward_only(xs, h)
        return _Sequence.apply(q, k, v, w, b, g, h)

    return call
