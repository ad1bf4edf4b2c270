"""Serving entry points of the GDN-2 operator on the HIP kernels: the single-token decode step
and the forward-only prefill with document resets.

Interface: the reference's inference module as of v0.3.1, whose source is inlined in
``notebooks/gdn2_v031_stage2_tpu.ipynb`` (cell 1, ``INFERENCE_V031``; v0.3.0 in
``notebooks/gdn2_v03_tpu_eval.ipynb``): ``LayerInputs``, ``decode_step`` and
``chunk_forward_inference`` with its argument names, defaults, validation order and error
messages.  Tensors are torch tensors on a ROCm device and dtypes are torch dtypes
(``torch.float32`` / ``torch.bfloat16``) where the reference takes jnp ones.

Kernels: ``decode_step`` and the prefill's tail (the tokens after its last full chunk) run the
token-recurrence kernel (``gdn2_decode``); the prefill's full chunks run the residual-free
forward with per-chunk state resets (``gdn2_fwd_reset``: the training forward's kernels, the
scan zeroing the state entering every chunk whose document differs from the previous chunk's).

Two cases where the reference's code departs from its own documented contract ("a document
boundary resets the state"; "initial_state is assumed to belong to the first chunk's
document") follow the contract here: in sequences longer than ``cfg.max_chunks_per_call``
chunks, the reference's kernel compares the first segment's chunk ids in every later segment
(its padded id block is not offset by the segment start); and with ``segment_ids`` on a
sequence shorter than one chunk it compares every token's id with 0 instead of with the
previous token's.  Here a chunk (or tail token) resets exactly when its document id differs
from the previous chunk's (token's).
"""
from __future__ import annotations

import ctypes
import dataclasses as _dc

import torch

from . import _lib
from .pipeline import _check_device

__all__ = ["decode_step", "chunk_forward_inference", "LayerInputs"]

_STATE_DTYPES = {torch.float32: 0, torch.bfloat16: 1, "float32": 0, "bfloat16": 1}


@_dc.dataclass(frozen=True)
class LayerInputs:
    """Named input container (reference ``LayerInputs``): q/k (B, H, Dk); v/w (B, Hv, Dv);
    g (B, H, Dk) per-token log-decay (<= 0); b (B, H, Dk).  Both entry points accept it instead
    of six positional tensors."""
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    w: torch.Tensor
    b: torch.Tensor
    g: torch.Tensor

    def validate(self, Dk: int, Dv: int):
        B = self.q.shape[0]
        want = {"q": (B, self.q.shape[1], Dk), "k": (B, self.q.shape[1], Dk),
                "v": (B, self.v.shape[1], Dv), "w": (B, self.v.shape[1], Dv),
                "b": (B, self.q.shape[1], Dk), "g": (B, self.q.shape[1], Dk)}
        for name, arr in (("q", self.q), ("k", self.k), ("v", self.v),
                          ("w", self.w), ("b", self.b), ("g", self.g)):
            if tuple(arr.shape) != want[name]:
                raise ValueError(f"{name}: expected {want[name]}, got {tuple(arr.shape)}")

    def as_tuple(self):
        return (self.q, self.k, self.v, self.w, self.b, self.g)


def _state_code(state_dtype):
    if state_dtype not in _STATE_DTYPES:
        raise ValueError(f"state_dtype must be float32 or bfloat16, got {state_dtype}")
    return _STATE_DTYPES[state_dtype]


def _torch_dtype(code):
    return torch.bfloat16 if code else torch.float32


def _inputs_for_kernel(ts):
    """The six inputs as the kernels take them: bfloat16 bits when all six are bfloat16 (widened
    to fp32 on load, the same values as the reference's up-front cast), fp32 otherwise."""
    if all(t.dtype == torch.bfloat16 for t in ts):
        return [t.contiguous() for t in ts], 1
    return [t.to(torch.float32).contiguous() for t in ts], 0


def _same_shape(ts, names, shape):
    for t, n in zip(ts, names):
        if tuple(t.shape) != tuple(shape):
            raise ValueError(f"{n}.shape={tuple(t.shape)} differs from q.shape={tuple(shape)}")
        if not t.is_floating_point():
            raise TypeError(f"{n} must be a floating-point tensor")


def _check_head_dim(D):
    if D not in (64, 128):
        raise ValueError(f"D={D}: the HIP kernels support head dimensions 64 and 128")


def _aligned(t):
    """The kernel reads 4 consecutive elements per access: a tensor whose first element is not
    16-byte aligned (a view at an odd offset) is copied."""
    return t if t is None or t.data_ptr() % 16 == 0 else t.clone()


def _run_decode(xs, in_dtype, B, H, D, n_tok, seq_ld, scale, state_in, state_code, o, out_code,
                reset=None, fuse=False, a_log=None, dt_bias=None, tau=None, offset=0):
    dev = xs[0].device
    xs = [_aligned(x) for x in xs]
    state_in = _aligned(state_in)
    if o.data_ptr() % 16:
        raise ValueError("o must be 16-byte aligned")
    state_out = torch.empty((B, H, D, D), dtype=_torch_dtype(state_code), device=dev)
    dd = _lib.Gdn2DecodeDesc(B, H, D, n_tok, seq_ld, in_dtype, out_code, state_code, int(fuse),
                             int(tau is not None), float(scale), float(tau) if tau is not None else 0.0)
    L_ = _lib.lib()
    with torch.cuda.device(dev):
        _lib.check(L_.gdn2_decode(ctypes.byref(dd), *(_lib.ptr(x, offset) for x in xs), _lib.ptr(a_log),
                                  _lib.ptr(dt_bias), _lib.ptr(reset), _lib.ptr(state_in), _lib.ptr(o, offset),
                                  _lib.ptr(state_out), _lib.stream_handle(dev)), "gdn2_decode")
    return state_out


def decode_step(q=None, k=None, v=None, w=None, b=None, g=None, state=None,
                scale: float = 1.0, reset=None, state_dtype=torch.float32,
                stability_tau=None, fuse_prologue: bool = False, a_log=None,
                dt_bias=None, inputs: "LayerInputs | None" = None, cfg=None):
    """Single-token recurrence for serving (reference ``decode_step``).

    q, k, v, w, b, g: (B, H, D), g this token's log-decay (positive values act as 0, as in
    token_serial_ref); state (B, H, D, D).  reset: (B,) -- rows whose value is > 0 after an
    integer cast start from a zero state.  fuse_prologue: q, k raw (l2-normalised in the kernel),
    b, w raw logits (sigmoid) and g the raw gate, g = -exp(a_log[h]) * softplus(g + dt_bias[d]),
    with a_log (H,) and dt_bias (D,).  stability_tau: cap on each head's Frobenius norm of the
    new state.  NaN / +-Inf entries of the new state and of o become 0.

    Returns (o (B, H, D) in q's dtype, new_state (B, H, D, D) in state_dtype).  Compute is fp32;
    the incoming state is first cast to state_dtype (as the reference does)."""
    if inputs is not None:
        q, k, v, w, b, g = inputs.as_tuple()
    if q is None or state is None:
        raise ValueError("pass either inputs=LayerInputs(...) or q,k,v,w,b,g,state")
    bsz, H, D = q.shape
    if not isinstance(scale, (int, float)) or isinstance(scale, torch.Tensor):
        raise ValueError(
            "scale must be a concrete Python float (B4): traced values cannot "
            "enter the kernel; pass it as a compile-time constant")
    if stability_tau is not None and not isinstance(stability_tau, (int, float)):
        raise ValueError(
            "stability_tau must be a concrete Python float (B4)")
    if tuple(state.shape) != (bsz, H, D, D):
        raise ValueError(f"state must be (B,H,D,D), got {tuple(state.shape)}")
    sc = _state_code(state_dtype)
    rst = None
    if reset is not None:
        rst = torch.as_tensor(reset).reshape(bsz).to(torch.int32) > 0
    if fuse_prologue:
        if a_log is None or dt_bias is None:
            raise ValueError(
                "fuse_prologue=True requires a_log (H,) and dt_bias (K,) from "
                "the checkpoint: the kernel then computes "
                "g = -exp(A_log) * softplus(g_raw + dt_bias) in-kernel")
        a_log = torch.as_tensor(a_log).reshape(H)
        dt_bias = torch.as_tensor(dt_bias).reshape(D)
    ts = (q, k, v, w, b, g)
    _same_shape(ts, "qkvwbg", (bsz, H, D))
    if q.numel() == 0:
        raise ValueError(f"empty input q.shape={tuple(q.shape)}: B, H and D must be positive")
    _check_head_dim(D)
    _check_device(q)
    dev = q.device
    for t, n in zip(ts[1:] + (state,), ("k", "v", "w", "b", "g", "state")):
        if t.device != dev:
            raise ValueError(f"{n} is on {t.device}, q on {dev}")
    xs, in_dtype = _inputs_for_kernel(ts)
    st = state.to(_torch_dtype(sc)).contiguous()
    out_code = 1 if q.dtype == torch.bfloat16 else 0
    o = torch.empty((bsz, H, D), dtype=_torch_dtype(out_code), device=dev)
    flags = None if rst is None else rst.to(device=dev, dtype=torch.uint8).contiguous()
    if fuse_prologue:
        a_log = a_log.to(device=dev, dtype=torch.float32).contiguous()
        dt_bias = dt_bias.to(device=dev, dtype=torch.float32).contiguous()
    new = _run_decode(xs, in_dtype, bsz, H, D, 1, 1, scale, st, sc, o, out_code, reset=flags,
                      fuse=fuse_prologue, a_log=a_log, dt_bias=dt_bias, tau=stability_tau)
    if o.dtype != q.dtype:
        o = o.to(q.dtype)
    return o, new


def _segment_ids_from_cu_seqlens(cu_seqlens, bsz, L, device):
    """cu_seqlens: 1-D (shared by every row) or (B, n_docs + 1) token offsets; a boundary token
    starts its document (reference INFERENCE_V031, the A3 conversion)."""
    cs = torch.as_tensor(cu_seqlens, device=device)
    if cs.dim() == 1:
        cs = cs[None, :].expand(bsz, cs.shape[0])
    n_int = cs.shape[1] - 2
    if n_int <= 0:
        return torch.zeros((bsz, L), dtype=torch.int32, device=device)
    bounds = cs[:, 1:-1]
    pos = torch.arange(L, device=device)
    return (pos[None, :, None] >= bounds[:, None, :]).sum(dim=-1).to(torch.int32)


def chunk_forward_inference(q=None, k=None, v=None, w=None, b=None, g=None,
                            scale: float = 1.0, cfg=None,
                            h0=None, segment_ids=None, cu_seqlens=None,
                            state_dtype=torch.float32, stability_tau=None,
                            inputs: "LayerInputs | None" = None):
    """Forward-only prefill (reference ``chunk_forward_inference``): returns (o, h_final) only.

    Head-major (B, H, L, D) inputs of any length L: the full chunks (L // cfg.bt of them) run the
    chunkwise forward, the remaining L % cfg.bt tokens the token recurrence (decode steps, the
    state rounded to state_dtype after each).  g is clamped to <= 0; min(g) below -cfg.g_max
    raises.  segment_ids (B, L): document ids; a chunk whose document differs from the previous
    chunk's starts from a zero state, and a document boundary inside a full chunk raises (the
    tail takes per-token boundaries).  cu_seqlens: 1-D or (B, n_docs + 1) token offsets instead
    of segment_ids.  h0 belongs to the first chunk's document.  stability_tau: cap on each head's
    Frobenius norm of the returned state.  o is float32; h_final is returned in state_dtype."""
    if inputs is not None:
        q, k, v, w, b, g = inputs.as_tuple()
    if q.dim() != 4:
        raise ValueError(f"expected (B,H,L,D) inputs, got q.shape={tuple(q.shape)}")
    bsz, H, L, D = q.shape
    _same_shape((q, k, v, w, b, g), "qkvwbg", (bsz, H, L, D))
    if bsz == 0 or H == 0 or D == 0:
        raise ValueError(f"empty input q.shape={tuple(q.shape)}: B, H and D must be positive")
    if h0 is not None and tuple(h0.shape) != (bsz, H, D, D):
        raise ValueError(f"h0.shape={tuple(h0.shape)} must be {(bsz, H, D, D)}")
    sc = _state_code(state_dtype)
    bt = cfg.bt
    n_full = L // bt
    L_full = n_full * bt
    r_tail = L - L_full
    scale = float(scale)
    dev = q.device
    g_max_abs = float(cfg.g_max)
    # The domain of g and the document boundaries are checked on the device and read back in one
    # synchronisation; g is clamped to <= 0 (as on the decode path) only when some g > 0.
    stats = []
    if L > 0:
        g_lo, g_hi = torch.aminmax(g)
        stats += [g_lo.float(), g_hi.float()]
    bad = None
    if segment_ids is not None and n_full > 0:
        seg_tok = torch.as_tensor(segment_ids, device=dev).reshape(bsz, L)[:, :L_full]
        per_chunk_first = seg_tok[:, ::bt]
        same = seg_tok.reshape(bsz, n_full, bt) == per_chunk_first[:, :, None]
        bad = ~same.all(dim=-1)
        stats.append(bad.any().float().to(dev))
    both = segment_ids is not None and cu_seqlens is not None
    if cu_seqlens is not None and not both:
        segment_ids = _segment_ids_from_cu_seqlens(cu_seqlens, bsz, L, dev)
    seg = None if segment_ids is None or both else torch.as_tensor(segment_ids, device=dev).reshape(bsz, L)
    # the reset bytes are formed before the synchronisation, so that the device is not left idle
    # while the host builds them after it
    flags = tflags = None
    if seg is not None and n_full > 0:
        sc_ids = seg[:, :L_full:bt]                                   # (B, n_full) id at each chunk start
        chg = torch.zeros_like(sc_ids, dtype=torch.bool)
        chg[:, 1:] = sc_ids[:, 1:] != sc_ids[:, :-1]
        per64 = torch.zeros((bsz, L_full // 64), dtype=torch.uint8, device=dev)
        per64[:, ::bt // 64] = chg.to(torch.uint8)                    # the chunk's first 64-token half
        flags = per64[:, None, :].expand(bsz, H, L_full // 64).contiguous()
    if seg is not None and r_tail > 0:
        tail = seg[:, L_full:]
        prev = seg[:, L_full - 1:L - 1] if L_full > 0 else torch.cat([tail[:, :1], tail[:, :-1]], dim=1)
        tflags = (tail != prev).to(torch.uint8).contiguous()
    vals = torch.stack([x.to(dev) for x in stats]).tolist() if stats else []
    # errors in the reference's order: g's domain, a boundary inside a chunk, both id forms
    if L > 0:
        # the layer's domain is [-g_max, 0] (NaN compares false, as in the reference)
        if min(vals[0], 0.0) < -g_max_abs - 1e-6:
            raise ValueError(
                f"g outside the layer domain: min(g) < -g_max={g_max_abs} "
                "(the layer constructs g = -min(softplus(...), g_max); clamp or "
                "fix the projection before calling)")
        if vals[1] > 0:
            g = torch.clamp(g, max=0.0)
    if bad is not None and vals[-1] > 0:
        b_idx, c_idx = (int(x) for x in torch.nonzero(bad)[0])
        raise ValueError(
            f"document boundary inside chunk {c_idx} of batch row "
            f"{b_idx} (tokens start at {c_idx * bt}): split "
            "the sequence at document boundaries before calling "
            "chunk_forward_inference (chunk-granularity resets only)")
    if both:
        raise ValueError("pass either segment_ids or cu_seqlens, not both")

    h = None if h0 is None else h0.to(torch.float32)
    o = None
    if L > 0:
        _check_head_dim(D)
        _check_device(q)
        xs, in_dtype = _inputs_for_kernel((q, k, v, w, b, g))
        h = None if h is None else h.to(dev).contiguous()
        o = torch.empty((bsz, H, L, D), dtype=torch.float32, device=dev)
        L_ = _lib.lib()
        if n_full > 0:
            desc = _lib.make_desc(cfg, bsz, H, L_full, D, scale, seq_ld=L)
            hf = torch.empty((bsz, H, D, D), dtype=torch.float32, device=dev)
            with torch.cuda.device(dev):
                ws = torch.empty(L_.gdn2_fwd_workspace_bytes(ctypes.byref(desc), 0), dtype=torch.uint8, device=dev)
                _lib.check(L_.gdn2_fwd_reset(ctypes.byref(desc), in_dtype, *map(_lib.ptr, xs), _lib.ptr(h),
                                             _lib.ptr(flags), _lib.ptr(o), _lib.ptr(hf), _lib.ptr(ws),
                                             _lib.stream_handle(dev)), "gdn2_fwd_reset")
            h = hf
        if r_tail > 0:
            st = None if h is None else h.to(_torch_dtype(sc)).contiguous()
            h = _run_decode(xs, in_dtype, bsz, H, D, r_tail, L, scale, st, sc, o, 0, reset=tflags,
                            offset=L_full * D)
    if h is None:
        h = torch.zeros((bsz, H, D, D), dtype=torch.float32, device=dev)
    if stability_tau is not None:
        hf32 = h.to(torch.float32)
        nrm = torch.sqrt((hf32 ** 2).sum(dim=(-2, -1), keepdim=True))
        f = torch.minimum(torch.ones_like(nrm), stability_tau / torch.maximum(nrm, torch.full_like(nrm, 1e-12)))
        h = hf32 * f
    return o, h.to(_torch_dtype(sc))
