"""CPU oracle for the GDN-2 operator -- TEST INFRASTRUCTURE ONLY.

This module restates, in torch (float64 by default, any float dtype accepted), the
algorithm of the reference's pure-JAX chunked-WY oracle and the semantics of its Pallas
kernels.  Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker or the timed CPU baseline.  The product
path (``atomic_gdn2`` + the HIP library) never calls into this file.

Reference anchors (``/root/reference``):

* ``atomic_gdn2/precision.py:41-52``   exp_nonpos / exp_clipped / sanitize  -> ``sanitize`` etc.
* ``atomic_gdn2/precision.py:8-38``    dot modes (highest / bf16x3 / default) -> ``make_dot``
* ``atomic_gdn2/layout.py:4-15``       chunk reshapes, causal masks
* ``atomic_gdn2/reference/ref.py:8-14``   to_chunks / from_chunks / chunk_gc
* ``atomic_gdn2/reference/ref.py:25-49``  blr_scores_ref (one-level BLR, exact clipped diagonal)
* ``atomic_gdn2/reference/ref.py:52-76``  _micro_inv / ladder_inverse
* ``atomic_gdn2/reference/ref.py:79-87``  recompute_wy_ref
* ``atomic_gdn2/reference/ref.py:90-101`` inter_chunk_scan_ref
* ``atomic_gdn2/reference/ref.py:104-113`` forward_ref
* ``atomic_gdn2/reference/ref.py:116-130`` token_serial_ref
* ``atomic_gdn2/reference/ref.py:133-153`` b4_exact_f64_np
* ``atomic_gdn2/fwd/scores.py:16-84``  two-level BLR scores with BTL / lean diagonal (kernel A)
* ``atomic_gdn2/fwd/cd_slim.py:8-31``  fused WY recompute + scan (kernel C+D)
* ``atomic_gdn2/bwd/mega.py:9-58``     fused analytic backward (B1..B5)
* ``atomic_gdn2/bwd/b4.py:7-97``       B4, the VJP of the two-level scores
* ``notebooks/gdn2_v031_stage2_tpu.ipynb`` cell 1 (``INFERENCE_V031``, the inference module
  inlined there): ``_decode_body`` / ``decode_step`` -> ``decode_step_ref``;
  ``_cd_inference_body`` / ``chunk_forward_inference`` -> ``chunk_forward_inference_ref``

Every function here is pinned by a test in ``tests/test_oracle_*.py`` (stored 80-digit
Decimal known-answer values, token-serial equality, closed forms, scipy triangular solves,
brute force on tiny inputs, finite differences, autograd-vs-analytic agreement).

Layout: the operator is head-major ``(B,H,L,D)``; chunked tensors are ``(B,H,nc,T,D)``.
The reference oracle's public functions take ``(B,L,H,D)``; ``forward_ref_blhd`` keeps that
convention, ``forward_ref`` here takes head-major tensors.
"""
from __future__ import annotations


from dataclasses import dataclass, replace

import numpy as np
import torch

__all__ = [
    "OracleCfg", "sanitize", "exp_nonpos", "exp_nonpos_grad", "exp_clipped", "make_dot", "bf16_round",
    "to_chunks", "from_chunks", "chunk_gc", "causal_masks",
    "blr_scores_ref", "btl_scores", "micro_inv", "ladder_inverse", "recompute_wy_ref",
    "inter_chunk_scan_ref", "forward_ref", "forward_ref_blhd", "token_serial_ref",
    "b4_exact_f64_np", "backward_mega_ref", "grad_ref", "wy_stage_ref",
    "decode_step_ref", "chunk_forward_inference_ref",
]


@dataclass(frozen=True)
class OracleCfg:
    """The config fields the reference oracle reads (``atomic_gdn2/config.py:31-50``)."""
    bt: int = 64
    score_bs: int = 64
    bs2: int = 32
    mb: int = 8
    diag: str = "btl"
    diff_clip: float = 20.0
    clip: float = 1e4
    wy_eps: float = 0.0
    dot_mode: str = "highest"
    solve_dot_mode: str = "highest"
    b3_dot_mode: str = "highest"

    def with_(self, **kw):
        return replace(self, **kw)

    @staticmethod
    def from_cfg(cfg) -> "OracleCfg":
        """Copy the oracle-relevant fields from any object that carries them."""
        names = OracleCfg.__dataclass_fields__.keys()
        return OracleCfg(**{n: getattr(cfg, n) for n in names if hasattr(cfg, n)})


# ----------------------------------------------------------------------------------------
# numerics helpers  (precision.py)
# ----------------------------------------------------------------------------------------
def sanitize(x, clip):
    """clip to +-clip, NaN -> 0, +-inf -> +-clip  (precision.py:51-52)."""
    return torch.nan_to_num(torch.clamp(x, -clip, clip), nan=0.0, posinf=clip, neginf=-clip)


def exp_nonpos(x):
    """exp(min(x,0)) and the 1{x<0} mask  (precision.py:41-44)."""
    return torch.exp(torch.clamp(x, max=0.0)), (x < 0.0).to(x.dtype)


def exp_nonpos_grad(x):
    """exp(min(x,0)) and its derivative mask 1{x<=0}: the gate on the dgc terms of the
    backward.  The reference's mega backward gates them with 1{x<0} (bwd/mega.py:25-26,32,
    47-48) although precision.py:42-43 states that this mask must not gate dgc terms
    (x == 0 on flat gc segments); its B4 drops the masks for that reason (bwd/b4.py:1,66).
    In fp32, gl - gc rounds to exactly 0 wherever the later gates of the chunk are below half
    an ulp of gc, and 1{x<0} then drops those rows' terms although the true x is negative.
    1{x<=0} equals 1 on the log-decay domain (g <= 0) and 0 for x > 0.  At an exact tie
    x == 0 (a token with g == 0 exactly) three conventions differ: the reference kernel's
    1{x<0} gives 0, JAX autograd of the reference's forward_ref gives 1/2 (jnp.minimum splits a
    tie), and this oracle and the HIP backward give 1 (torch's derivative of clamp(x, max=0)).
    No reference fixture has g == 0, so dg there is parity unpinned; inputs with g < 0 strictly
    (every benchmark input) never reach a tie except through fp32 rounding of gl - gc, where 1
    is the value of the untied neighbourhood.  On the last row x = gl - gc is identically 0 and
    its term cancels against the last-row sum."""
    return torch.exp(torch.clamp(x, max=0.0)), (x <= 0.0).to(x.dtype)


def exp_clipped(x, lo, hi):
    """exp(clip(x,lo,hi)) and the in-range mask  (precision.py:47-48)."""
    return torch.exp(torch.clamp(x, lo, hi)), ((x >= lo) & (x <= hi)).to(x.dtype)


def bf16_round(x):
    """Round to bfloat16 (round-to-nearest-even) and return in x's dtype.

    For float64 inputs the value is first rounded to float32, as the reference's float32
    arrays would be, then to bfloat16.
    """
    return x.to(torch.float32).to(torch.bfloat16).to(x.dtype)


def _split_bf16(x):
    """hi = bf16(x), lo = bf16(x - hi)  (precision.py:8-11)."""
    hi = bf16_round(x)
    lo = bf16_round(x.to(torch.float32).to(x.dtype) - hi)
    return hi, lo


def make_dot(mode: str):
    """Matrix product under a dot mode  (precision.py:14-31).

    ``highest``: the plain product in the working dtype.
    ``bf16x3``:  hi*hi + hi*lo + lo*hi with bf16-rounded parts, exact products.
    ``default``: one pass on bf16-rounded operands.
    """
    if mode == "highest":
        return torch.matmul
    if mode == "bf16x3":
        def dot3(a, b):
            ah, al = _split_bf16(a)
            bh, bl = _split_bf16(b)
            return torch.matmul(ah, bh) + torch.matmul(ah, bl) + torch.matmul(al, bh)
        return dot3
    if mode == "default":
        return lambda a, b: torch.matmul(bf16_round(a), bf16_round(b))
    raise ValueError(mode)


# ----------------------------------------------------------------------------------------
# layout  (layout.py, ref.py:8-14)
# ----------------------------------------------------------------------------------------
def to_chunks(t, bt):
    """(B,H,L,D) -> (B,H,nc,bt,D), a pure reshape (layout.py:4-7)."""
    B, H, L, D = t.shape
    return t.reshape(B, H, L // bt, bt, D)


def from_chunks(t):
    B, H, nc, bt, D = t.shape
    return t.reshape(B, H, nc * bt, D)


def chunk_gc(g_ch):
    """In-chunk cumulative log-decay (ref.py:14)."""
    return torch.cumsum(g_ch, dim=-2)


def causal_masks(T, dtype=torch.float64):
    i = torch.arange(T)
    return (i[:, None] >= i[None, :]).to(dtype), (i[:, None] > i[None, :]).to(dtype)


def _place(block, p0, p1, T):
    """Embed a (...,r,p1-p0) block into (...,r,T) columns (ref.py:17-22)."""
    lead = block.shape[:-1]
    out = block.new_zeros(lead + (T,))
    out = out.clone()
    out[..., p0:p1] = block
    return out


# ----------------------------------------------------------------------------------------
# scores
# ----------------------------------------------------------------------------------------
def blr_scores_ref(q, k, b, gc, scale, cfg: OracleCfg):
    """Oracle scores (ref.py:27-51): one level of block-local rescaling at ``score_bs`` for
    the rows below each outer block, and an exact per-element ``exp(clip(dG,+-diff_clip))``
    on the outer diagonal blocks.  Inputs (...,T,D).  Returns Aqk (causal), Akk (strict)."""
    T, bs, dc = cfg.bt, cfg.score_bs, cfg.diff_clip
    dt = q.dtype
    causal, strict = causal_masks(T, dt)
    idx = torch.arange(T)
    bk = b * k
    rq, rk = [], []
    for p in range(T // bs):
        p0, p1 = p * bs, (p + 1) * bs
        r = gc[..., p0, :]
        a, _ = exp_nonpos(gc[..., p0:p1, :] - r[..., None, :])
        if p0 > 0:
            c, _ = exp_nonpos(r[..., None, :] - gc)
            kt = k * c
            before = (idx < p0).to(dt)
            oq = scale * torch.einsum("...id,...jd->...ij", q[..., p0:p1, :] * a, kt) * before
            ok = torch.einsum("...id,...jd->...ij", bk[..., p0:p1, :] * a, kt) * before
        else:
            oq = q.new_zeros(q.shape[:-2] + (bs, T))
            ok = oq
        gd = gc[..., p0:p1, :]
        E, _ = exp_clipped(gd[..., :, None, :] - gd[..., None, :, :], -dc, dc)
        dq_ = scale * torch.einsum("...id,...ijd,...jd->...ij", q[..., p0:p1, :], E, k[..., p0:p1, :])
        dk_ = torch.einsum("...id,...ijd,...jd->...ij", bk[..., p0:p1, :], E, k[..., p0:p1, :])
        rq.append(oq + _place(dq_, p0, p1, T))
        rk.append(ok + _place(dk_, p0, p1, T))
    return (sanitize(torch.cat(rq, -2) * causal, cfg.clip),
            sanitize(torch.cat(rk, -2) * strict, cfg.clip))


def _btl_legs(gc, s0, s1):
    """Balanced two-leg factors of a diagonal block (fwd/scores.py:16-22)."""
    r = gc[..., s0, :]
    half = 0.5 * (gc[..., s0, :] - gc[..., s1 - 1, :])
    ea = torch.exp((gc[..., s0:s1, :] - r[..., None, :]) + half[..., None, :])
    ec = torch.exp((r[..., None, :] - gc[..., s0:s1, :]) - half[..., None, :])
    return ea, ec


def btl_scores(q, k, b, gc, scale, cfg: OracleCfg, dot=None):
    """Kernel-A semantics (fwd/scores.py:39-84): two-level block-local rescaling with anchor
    rows at each ``score_bs`` and ``bs2`` block start, BTL (or lean) diagonal ``bs2`` blocks,
    causal/strict masks and ``sanitize``.  Inputs (...,T,D)."""
    T, bs, bs2, dc = cfg.bt, cfg.score_bs, cfg.bs2, cfg.diff_clip
    dot = dot or make_dot(cfg.dot_mode)
    dt = q.dtype
    causal, strict = causal_masks(T, dt)
    idx = torch.arange(T)
    bk = b * k
    tr = lambda x: x.transpose(-1, -2)
    Aq = q.new_zeros(q.shape[:-2] + (T, T))
    Ak = q.new_zeros(q.shape[:-2] + (T, T))
    for p in range(T // bs):
        p0, p1 = p * bs, (p + 1) * bs
        if p0 > 0:
            r1 = gc[..., p0, :]
            a1, _ = exp_nonpos(gc[..., p0:p1, :] - r1[..., None, :])
            c1, _ = exp_nonpos(r1[..., None, :] - gc)
            before = (idx < p0).to(dt)
            kt1 = k * c1
            l1q = scale * dot(q[..., p0:p1, :] * a1, tr(kt1)) * before
            l1k = dot(bk[..., p0:p1, :] * a1, tr(kt1)) * before
        else:
            l1q = q.new_zeros(q.shape[:-2] + (bs, T))
            l1k = l1q
        for kk in range(bs // bs2):
            q0, q1 = p0 + kk * bs2, p0 + (kk + 1) * bs2
            rowq = l1q[..., kk * bs2:(kk + 1) * bs2, :]
            rowk = l1k[..., kk * bs2:(kk + 1) * bs2, :]
            if kk > 0:
                r2 = gc[..., q0, :]
                a2, _ = exp_nonpos(gc[..., q0:q1, :] - r2[..., None, :])
                c2, _ = exp_nonpos(r2[..., None, :] - gc[..., p0:q0, :])
                kt2 = k[..., p0:q0, :] * c2
                rowq = rowq + _place(scale * dot(q[..., q0:q1, :] * a2, tr(kt2)), p0, q0, T)
                rowk = rowk + _place(dot(bk[..., q0:q1, :] * a2, tr(kt2)), p0, q0, T)
            if cfg.diag == "btl":
                ea, ec = _btl_legs(gc, q0, q1)
                kt = k[..., q0:q1, :] * ec
                bq = scale * dot(q[..., q0:q1, :] * ea, tr(kt))
                bkk = dot(bk[..., q0:q1, :] * ea, tr(kt))
            else:
                gd = gc[..., q0:q1, :]
                E, _ = exp_clipped(gd[..., :, None, :] - gd[..., None, :, :], -dc, dc)
                bq = scale * torch.sum(q[..., q0:q1, None, :] * E * k[..., None, q0:q1, :], -1)
                bkk = torch.sum(bk[..., q0:q1, None, :] * E * k[..., None, q0:q1, :], -1)
            Aq = Aq.clone()
            Ak = Ak.clone()
            Aq[..., q0:q1, :] = rowq + _place(bq, q0, q1, T)
            Ak[..., q0:q1, :] = rowk + _place(bkk, q0, q1, T)
    return sanitize(Aq * causal, cfg.clip), sanitize(Ak * strict, cfg.clip)


# ----------------------------------------------------------------------------------------
# WY inverse  (ref.py:54-78, fwd/solve.py:9-43)
# ----------------------------------------------------------------------------------------
def micro_inv(Tm):
    """Inverse of (I + Tm) for strictly lower Tm by row recursion  (ref.py:52-60):
    row_i = e_i - sum_j Tm[i,j] * row_j."""
    mb = Tm.shape[-1]
    eye = torch.eye(mb, dtype=Tm.dtype)
    rows = []
    for i in range(mb):
        acc = eye[i].expand(Tm.shape[:-2] + (mb,))
        for j in range(i):
            acc = acc - Tm[..., i, j, None] * rows[j]
        rows.append(acc)
    return torch.stack(rows, -2)


def ladder_inverse(S, eps, C, base, mode="highest"):
    """A = (I + (1-eps) S)^-1 by leaf inverses of size ``base`` and block doubling
    X <- [[top, 0], [-bot (S_l top), bot]]  (ref.py:63-76)."""
    dot = make_dot(mode)
    nb = C // base
    Se = S * (1.0 - eps)
    X = [micro_inv(Se[..., m * base:(m + 1) * base, m * base:(m + 1) * base]) for m in range(nb)]
    b_ = base
    while b_ < C:
        n2, new = 2 * b_, []
        for m in range(C // n2):
            top, bot = X[2 * m], X[2 * m + 1]
            i0 = m * n2
            mid = dot(Se[..., i0 + b_:i0 + n2, i0:i0 + b_], top)
            ll = -dot(bot, mid)
            z = torch.zeros_like(ll)
            new.append(torch.cat([torch.cat([top, z], -1), torch.cat([ll, bot], -1)], -2))
        X, b_ = new, n2
    return X[0]


# ----------------------------------------------------------------------------------------
# WY recompute, scan, forward  (ref.py:79-113)
# ----------------------------------------------------------------------------------------
def recompute_wy_ref(q, k, v, w, b, gc, A, cfg: OracleCfg, dot=None):
    dot = dot or torch.matmul
    egc, _ = exp_nonpos(gc)
    wp = dot(A, b * k * egc)
    u = dot(A, w * v)
    gl = gc[..., -1, :]
    ekg, _ = exp_nonpos(gl[..., None, :] - gc)
    c = cfg.clip
    return sanitize(wp, c), sanitize(u, c), sanitize(k * ekg, c), sanitize(q * egc, c), gl


def inter_chunk_scan_ref(Aqk, wp, u, kg, qg, gc_last, scale, h0, cfg: OracleCfg, dot=None, reset=None):
    """Sequential scan over the chunk axis (-3); returns o, h_final, h_pre_all, v_new_all.
    reset (B, nc) bool, optional: the state entering chunk i of batch row b is zero where set
    (the document resets of the inference prefill, INFERENCE_V031 _cd_inference_body)."""
    dot = dot or torch.matmul
    c = cfg.clip
    nc = Aqk.shape[-3]
    h = h0
    os_, hp, vn = [], [], []
    for i in range(nc):
        if reset is not None:
            h = torch.where(reset[:, i][:, None, None, None], torch.zeros_like(h), h)
        Aq, wp_, u_, kg_, qg_, gl = (x[..., i, :, :] if x.dim() == Aqk.dim() else x[..., i, :]
                                     for x in (Aqk, wp, u, kg, qg, gc_last))
        v_new = u_ - dot(wp_, h)
        o = scale * dot(qg_, h) + dot(Aq, v_new)
        dec, _ = exp_nonpos(gl)
        hp.append(h)
        vn.append(v_new)
        os_.append(sanitize(o, c))
        h = sanitize(h * dec[..., :, None] + dot(kg_.transpose(-1, -2), v_new), c)
    return torch.stack(os_, -3), h, torch.stack(hp, -3), torch.stack(vn, -3)


def forward_ref(q, k, v, w, b, g, scale, h0, cfg: OracleCfg):
    """Head-major (B,H,L,D) restatement of ``forward_ref`` (ref.py:106-115): exact-diagonal
    scores, ladder inverse at 'highest', WY recompute, inter-chunk scan.  Autograd-transparent.
    Returns o (B,H,L,D), h_final (B,H,D,D)."""
    ch = lambda t: to_chunks(t, cfg.bt)
    qr, kr, vr, wr, br, gr = map(ch, (q, k, v, w, b, g))
    gc = chunk_gc(gr)
    Aqk, Akk = blr_scores_ref(qr, kr, br, gc, scale, cfg)
    A = sanitize(ladder_inverse(Akk, cfg.wy_eps, cfg.bt, cfg.mb, "highest"), cfg.clip)
    wp, u, kg, qg, gl = recompute_wy_ref(qr, kr, vr, wr, br, gc, A, cfg)
    if h0 is None:
        h0 = q.new_zeros(q.shape[:2] + (q.shape[-1], q.shape[-1]))
    o, hf, _, _ = inter_chunk_scan_ref(Aqk, wp, u, kg, qg, gl, scale, h0, cfg)
    return from_chunks(o), hf


def forward_ref_blhd(q, k, v, w, b, g, scale, h0, cfg: OracleCfg):
    """The reference oracle's own (B,L,H,D) convention (ref.py:106-115)."""
    sw = lambda t: t.transpose(1, 2)
    o, hf = forward_ref(*(sw(t) for t in (q, k, v, w, b, g)), scale, h0, cfg)
    return sw(o), hf


def wy_stage_ref(q, k, v, w, b, g, scale, cfg: OracleCfg):
    """Per-chunk intermediates of the forward in kernel semantics (two-level scores with the
    configured diagonal, ladder inverse in ``solve_dot_mode``, WY recompute in ``dot_mode``):
    dict of gc, Aqk, Akk, A, wp, u, kg, qg, gc_last, all (B,H,nc,...)."""
    ch = lambda t: to_chunks(t, cfg.bt)
    qr, kr, vr, wr, br, gr = map(ch, (q, k, v, w, b, g))
    gc = chunk_gc(gr)
    Aqk, Akk = btl_scores(qr, kr, br, gc, scale, cfg)
    A = sanitize(ladder_inverse(Akk, cfg.wy_eps, cfg.bt, cfg.mb, cfg.solve_dot_mode), cfg.clip)
    wp, u, kg, qg, gl = recompute_wy_ref(qr, kr, vr, wr, br, gc, A, cfg, make_dot(cfg.dot_mode))
    return dict(gc=gc, Aqk=Aqk, Akk=Akk, A=A, wp=wp, u=u, kg=kg, qg=qg, gc_last=gl)


def token_serial_ref(q, k, v, g, b, w, scale, h0=None):
    """Token recurrence on (B,L,H,D) inputs (ref.py:118-132); note the (q,k,v,g,b,w) order:
    h <- diag(exp(min(g,0))) h;  v_new = w*v - h^T (b*k);  h += k v_new^T;  o = h^T (s q)."""
    B, L, H, D = q.shape
    if h0 is None:
        h0 = q.new_zeros((B, H, D, D))
    alpha = torch.exp(torch.clamp(g, max=0.0))
    h = h0
    outs = []
    for t in range(L):
        h = h * alpha[:, t, :, :, None]
        erase = torch.einsum("bhd,bhdv->bhv", b[:, t] * k[:, t], h)
        v_new = w[:, t] * v[:, t] - erase
        h = h + torch.einsum("bhd,bhv->bhdv", k[:, t], v_new)
        outs.append(torch.einsum("bhdv,bhd->bhv", h, q[:, t] * scale))
    return torch.stack(outs, 1), h


# ----------------------------------------------------------------------------------------
# Inference entry points (reference notebooks/gdn2_v031_stage2_tpu.ipynb, cell 1, INFERENCE_V031)
# ----------------------------------------------------------------------------------------
def _nan_to_num0(x):
    return torch.where(torch.isfinite(x), x, torch.zeros_like(x))


def decode_step_ref(q, k, v, w, b, g, state, scale, reset=None, state_bf16=False, stability_tau=None,
                    fuse_prologue=False, a_log=None, dt_bias=None, out_bf16=False):
    """One token of the recurrence, (B,H,D) inputs, (B,H,D,D) state (INFERENCE_V031
    _decode_body / decode_step): the incoming state cast to the state dtype and zeroed for reset
    rows; optional prologue (q, k l2-normalised with eps 1e-6, b, w sigmoid, g = -exp(a_log)
    softplus(g + dt_bias)); h = diag(e^min(g,0)) S; v_new = w v - h^T (b k); h += k v_new^T;
    o = h^T (s q); optional per-head Frobenius cap; NaN/Inf -> 0 in h and o; o and the state
    rounded to their storage dtypes.  Computes in the inputs' dtype (float64 for the checks)."""
    st = bf16_round(state) if state_bf16 else state
    if reset is not None:
        st = torch.where(reset.reshape(-1)[:, None, None, None] > 0, torch.zeros_like(st), st)
    if fuse_prologue:
        q = q / torch.sqrt((q * q).sum(-1, keepdim=True) + 1e-6)
        k = k / torch.sqrt((k * k).sum(-1, keepdim=True) + 1e-6)
        b = torch.sigmoid(b)
        w = torch.sigmoid(w)
        g = -torch.exp(a_log)[None, :, None] * torch.nn.functional.softplus(g + dt_bias[None, None, :])
    h = st * torch.exp(torch.clamp(g, max=0.0))[..., None]
    erase = ((b * k)[..., None] * h).sum(-2)
    v_new = w * v - erase
    h = h + k[..., None] * v_new[..., None, :]
    o = (h * (q * scale)[..., None]).sum(-2)
    if stability_tau is not None:
        nrm = torch.sqrt((h * h).sum((-2, -1)))
        f = torch.minimum(torch.ones_like(nrm), stability_tau / torch.maximum(nrm, torch.full_like(nrm, 1e-12)))
        h = h * f[..., None, None]
    h = _nan_to_num0(h)
    o = _nan_to_num0(o)
    return (bf16_round(o) if out_bf16 else o), (bf16_round(h) if state_bf16 else h)


def chunk_forward_inference_ref(q, k, v, w, b, g, scale, cfg: OracleCfg, h0=None, segment_ids=None,
                                state_bf16=False, stability_tau=None):
    """Forward-only prefill (INFERENCE_V031 chunk_forward_inference) on head-major (B,H,L,D)
    inputs of any length: g clamped to <= 0; the L // bt full chunks in kernel semantics
    (wy_stage_ref + inter_chunk_scan_ref) with the state zeroed entering every chunk whose
    document id (segment_ids (B,L) at the chunk's first token) differs from the previous
    chunk's; the L % bt tail token by token (decode_step_ref, the state rounded to the state
    dtype after each token) with a reset wherever the id differs from the previous token's;
    then the optional per-head Frobenius cap.  Returns o, h_final (state dtype applied)."""
    B, H, L, D = q.shape
    bt = cfg.bt
    n_full = L // bt
    L_full = n_full * bt
    g = torch.clamp(g, max=0.0)
    h = q.new_zeros((B, H, D, D)) if h0 is None else h0.to(q.dtype)
    outs = []
    if n_full > 0:
        sl = lambda t: t[:, :, :L_full]
        st = wy_stage_ref(*(sl(t) for t in (q, k, v, w, b, g)), scale, cfg)
        reset = None
        if segment_ids is not None:
            ids = segment_ids[:, :L_full:bt]
            reset = torch.zeros_like(ids, dtype=torch.bool)
            reset[:, 1:] = ids[:, 1:] != ids[:, :-1]
        o, h, _, _ = inter_chunk_scan_ref(st["Aqk"], st["wp"], st["u"], st["kg"], st["qg"], st["gc_last"],
                                          scale, h, cfg, make_dot(cfg.dot_mode), reset=reset)
        outs.append(from_chunks(o))
    if L > L_full:
        h = bf16_round(h) if state_bf16 else h
        for t in range(L_full, L):
            rst = None
            if segment_ids is not None:
                prev = segment_ids[:, t - 1] if t > 0 else segment_ids[:, t]
                rst = (segment_ids[:, t] != prev).to(torch.int32)
            o_t, h = decode_step_ref(q[:, :, t], k[:, :, t], v[:, :, t], w[:, :, t], b[:, :, t], g[:, :, t],
                                     h, scale, reset=rst, state_bf16=state_bf16)
            outs.append(o_t[:, :, None])
    o = torch.cat(outs, 2) if outs else None
    if stability_tau is not None:
        nrm = torch.sqrt((h * h).sum((-2, -1), keepdim=True))
        h = h * torch.minimum(torch.ones_like(nrm), stability_tau / torch.maximum(nrm, torch.full_like(nrm, 1e-12)))
    return o, (bf16_round(h) if state_bf16 else h)


def b4_exact_f64_np(q, k, b, gc, dAq, dAk, scale, clip=1e4, dc=20.0, dblk=8):
    """Exact, non-factorised B4 for one chunk (T,D) in numpy float64 (ref.py:133-153).
    Returns dq, dk (incl. d(bk)*b), db, dgc, all sanitized."""
    f = lambda x: np.asarray(x.detach().cpu().numpy() if torch.is_tensor(x) else x, np.float64)
    q, k, b, gc, dAq, dAk = map(f, (q, k, b, gc, dAq, dAk))
    T, D = q.shape
    i = np.arange(T)
    dAq = dAq * (i[:, None] >= i[None, :])
    dAk = dAk * (i[:, None] > i[None, :])
    bk = b * k
    dq = np.zeros((T, D)); dbk = np.zeros((T, D)); dk = np.zeros((T, D)); dgc = np.zeros((T, D))
    for d0 in range(0, D, dblk):
        d1 = min(d0 + dblk, D)
        diff = gc[:, None, d0:d1] - gc[None, :, d0:d1]
        cm = ((diff >= -dc) & (diff <= dc)).astype(np.float64)
        E = np.exp(np.clip(diff, -dc, dc))
        kd = k[None, :, d0:d1]
        dq[:, d0:d1] = scale * np.sum(dAq[:, :, None] * E * kd, axis=1)
        dbk[:, d0:d1] = np.sum(dAk[:, :, None] * E * kd, axis=1)
        dk[:, d0:d1] = (scale * np.sum(dAq[:, :, None] * E * q[:, None, d0:d1], axis=0)
                        + np.sum(dAk[:, :, None] * E * bk[:, None, d0:d1], axis=0))
        wgt = ((dAq[:, :, None] * (scale * q)[:, None, d0:d1] + dAk[:, :, None] * bk[:, None, d0:d1])
               * k[None, :, d0:d1] * E * cm)
        dgc[:, d0:d1] = np.sum(wgt, axis=1) - np.sum(wgt, axis=0)
    san = lambda x: np.nan_to_num(np.clip(x, -clip, clip), nan=0.0, posinf=clip, neginf=-clip)
    return san(dq), san(dk + dbk * b), san(dbk * k), san(dgc)


# ----------------------------------------------------------------------------------------
# analytic backward in kernel semantics  (bwd/mega.py:9-58, bwd/b4.py:7-97)
# ----------------------------------------------------------------------------------------
def _b4_2l(q, k, b, gc, dAqk, dAkk, scale, cfg: OracleCfg, dot):
    """B4 (bwd/b4.py:45-97): VJP of the two-level scores for one set of chunks (...,T,D).
    dAqk / dAkk arrive masked (causal / strict).  No clamp masks on dgc terms."""
    T, bs, bs2, dc, c_ = cfg.bt, cfg.score_bs, cfg.bs2, cfg.diff_clip, cfg.clip
    dt = q.dtype
    idx = torch.arange(T)
    bk = b * k
    tr = lambda x: x.transpose(-1, -2)
    lead = q.shape[:-2]
    D = q.shape[-1]
    dk_g = q.new_zeros(lead + (T, D))
    dgc_g = q.new_zeros(lead + (T, D))
    dq_parts, dbk_parts = [], []

    def scat(x, lo, n_rows):
        out = x.new_zeros(lead + (n_rows, D)).clone()
        out[..., lo:lo + x.shape[-2], :] = x
        return out

    for p in range(T // bs):
        p0, p1 = p * bs, (p + 1) * bs
        dq_l = q.new_zeros(lead + (bs, D)); dbk_l = dq_l; dk_l = dq_l; dgc_l = dq_l
        before = (idx < p0).to(dt)
        if p0 > 0:
            r1 = gc[..., p0, :]
            a1, _ = exp_nonpos(gc[..., p0:p1, :] - r1[..., None, :])
            c1, _ = exp_nonpos(r1[..., None, :] - gc)
            qt1, bkt1 = q[..., p0:p1, :] * a1, bk[..., p0:p1, :] * a1
            kt1 = k * c1 * before[:, None]
            dMq1 = dAqk[..., p0:p1, :] * before
            dMk1 = dAkk[..., p0:p1, :] * before
            dqt1 = scale * dot(dMq1, kt1); dbkt1 = dot(dMk1, kt1)
            dkt1 = scale * dot(tr(dMq1), qt1) + dot(tr(dMk1), bkt1)
            dq_l = dq_l + dqt1 * a1; dbk_l = dbk_l + dbkt1 * a1
            dk_g = sanitize(dk_g + dkt1 * c1 * before[:, None], c_)
            dgc_g = sanitize(dgc_g - dkt1 * kt1, c_)
            dgc_l = dgc_l + (dqt1 * qt1 + dbkt1 * bkt1)
        for kk in range(bs // bs2):
            lo, hi = kk * bs2, (kk + 1) * bs2
            q0, q1 = p0 + lo, p0 + hi
            if kk > 0:
                r2 = gc[..., q0, :]
                a2, _ = exp_nonpos(gc[..., q0:q1, :] - r2[..., None, :])
                c2, _ = exp_nonpos(r2[..., None, :] - gc[..., p0:q0, :])
                qt2, bkt2 = q[..., q0:q1, :] * a2, bk[..., q0:q1, :] * a2
                kt2 = k[..., p0:q0, :] * c2
                dMq2, dMk2 = dAqk[..., q0:q1, p0:q0], dAkk[..., q0:q1, p0:q0]
                dqt2 = scale * dot(dMq2, kt2); dbkt2 = dot(dMk2, kt2)
                dkt2 = scale * dot(tr(dMq2), qt2) + dot(tr(dMk2), bkt2)
                dq_l = dq_l + scat(dqt2 * a2, lo, bs)
                dbk_l = dbk_l + scat(dbkt2 * a2, lo, bs)
                dk_l = dk_l + scat(dkt2 * c2, 0, bs)
                dgc_l = dgc_l + scat(-(dkt2 * kt2), 0, bs)
                dgc_l = dgc_l + scat(dqt2 * qt2 + dbkt2 * bkt2, lo, bs)
            qd, kd, bkd = q[..., q0:q1, :], k[..., q0:q1, :], bk[..., q0:q1, :]
            dMq, dMk = dAqk[..., q0:q1, q0:q1], dAkk[..., q0:q1, q0:q1]
            if cfg.diag == "btl":
                ea, ec = _btl_legs(gc, q0, q1)
                qt, bkt, kt = qd * ea, bkd * ea, kd * ec
                dqt = scale * dot(dMq, kt); dbkt = dot(dMk, kt)
                dkt = scale * dot(tr(dMq), qt) + dot(tr(dMk), bkt)
                dq_d, dbk_d, dk_d = dqt * ea, dbkt * ea, dkt * ec
            else:
                gd = gc[..., q0:q1, :]
                E = torch.exp(torch.clamp(gd[..., :, None, :] - gd[..., None, :, :], -dc, dc))
                Ek = E * kd[..., None, :, :]
                dq_d = scale * torch.sum(dMq[..., :, :, None] * Ek, -2)
                dbk_d = torch.sum(dMk[..., :, :, None] * Ek, -2)
                M = dMq[..., :, :, None] * (scale * qd)[..., :, None, :] + dMk[..., :, :, None] * bkd[..., :, None, :]
                dk_d = torch.sum(M * E, -3)
            dgc_d = qd * dq_d + bkd * dbk_d - kd * dk_d
            dq_l = dq_l + scat(dq_d, lo, bs)
            dbk_l = dbk_l + scat(dbk_d, lo, bs)
            dk_l = dk_l + scat(dk_d, lo, bs)
            dgc_l = dgc_l + scat(dgc_d, lo, bs)
        dq_parts.append(dq_l); dbk_parts.append(dbk_l)
        dk_g = sanitize(dk_g + scat(dk_l, p0, T), c_)
        dgc_g = sanitize(dgc_g + scat(dgc_l, p0, T), c_)
    dq_v = sanitize(torch.cat(dq_parts, -2), c_)
    dbk_v = sanitize(torch.cat(dbk_parts, -2), c_)
    return dq_v, sanitize(dk_g + dbk_v * b, c_), sanitize(dbk_v * k, c_), sanitize(dgc_g, c_)


def backward_mega_ref(q, k, v, w, b, g, A, Aqk, h_pre, v_new, do, dhf, scale, cfg: OracleCfg):
    """Analytic backward in kernel semantics (bwd/mega.py:9-58) on chunked tensors
    (B,H,nc,T,D); A/Aqk (B,H,nc,T,T), h_pre (B,H,nc,D,D), dhf (B,H,D,D).
    Returns dict dq,dk,db,dw,dv,dg (chunked) and dh0, plus per-chunk intermediates
    dv_new, dh_next, dAkk, dAqk for stage-level checks."""
    dot3 = make_dot(cfg.b3_dot_mode)
    dot_hi = make_dot(cfg.dot_mode)
    dot4 = make_dot("highest")
    T, c_ = cfg.bt, cfg.clip
    dt = q.dtype
    causal, strict = causal_masks(T, dt)
    idx = torch.arange(T)
    triu = (idx[:, None] <= idx[None, :]).to(dt)
    last = (idx == (T - 1)).to(dt)[:, None]
    tr = lambda x: x.transpose(-1, -2)
    gc_all = chunk_gc(g)
    nc = q.shape[-3]
    dh = dhf
    outs = {n: [None] * nc for n in ("dq", "dk", "db", "dw", "dv", "dg", "dv_new", "dh_next", "dAkk", "dAqk")}
    for c in range(nc - 1, -1, -1):
        sl = lambda x: x[..., c, :, :]
        qc, kc, bc_, wc, vc, gc = map(sl, (q, k, b, w, v, gc_all))
        Ac, Aqc, hp, vn, doc = map(sl, (A, Aqk, h_pre, v_new, do))
        gl = gc[..., T - 1, :]
        egc, mgc = exp_nonpos_grad(gc)
        ekg, mkg = exp_nonpos_grad(gl[..., None, :] - gc)
        kb = bc_ * kc * egc
        kg = sanitize(kc * ekg, c_)
        qg = sanitize(qc * egc, c_)
        wp = sanitize(dot_hi(Ac, kb), c_)
        dAqk = dot3(doc, tr(vn)) * causal
        dv_new = sanitize(dot3(tr(Aqc), doc) + dot3(kg, dh), c_)
        dec, mdec = exp_nonpos_grad(gl)
        dh_next = dh
        dh = sanitize(dot3(tr(qg), scale * doc) + dh * dec[..., :, None] - dot3(tr(wp), dv_new), c_)
        wv = wc * vc
        dqg = dot3(scale * doc, tr(hp))
        dwp = dot3(-dv_new, tr(hp))
        dkg = dot3(vn, tr(dh_next))
        dA = sanitize(dot3(dwp, tr(kb)) + dot3(dv_new, tr(wv)), c_)
        dkb = dot3(tr(Ac), dwp)
        dwv = dot3(tr(Ac), dv_new)
        tmp = sanitize(dot3(dA, tr(Ac)), c_)
        dAkk = sanitize((-dot3(tr(Ac), tmp) * (1.0 - cfg.wy_eps)) * strict, c_)
        dx = dkg * kg
        dq3 = dqg * egc
        dk3 = dkb * egc * bc_ + dkg * ekg
        db3 = dkb * egc * kc
        dgc3 = dkb * kb * mgc + dqg * qg * mgc - dx * mkg
        dgc_last = torch.sum(dx * mkg, -2) + dec * torch.sum(dh_next * hp, -1) * mdec
        dgc3 = sanitize(dgc3 + last * dgc_last[..., None, :], c_)
        dq4, dk4, db4, dgc4 = _b4_2l(qc, kc, bc_, gc, dAqk, dAkk * strict, scale, cfg, dot4)
        dg_ = dot4(triu, dgc3 + dgc4)
        outs["dq"][c] = sanitize(dq3 + dq4, c_)
        outs["dk"][c] = sanitize(dk3 + dk4, c_)
        outs["db"][c] = sanitize(db3 + db4, c_)
        outs["dw"][c] = sanitize(dwv * vc, c_)
        outs["dv"][c] = sanitize(dwv * wc, c_)
        outs["dg"][c] = sanitize(dg_, c_)
        outs["dv_new"][c] = dv_new
        outs["dh_next"][c] = dh_next
        outs["dAkk"][c] = dAkk
        outs["dAqk"][c] = dAqk
    res = {n: torch.stack(x, -3) for n, x in outs.items()}
    res["dh0"] = dh
    return res


def kernel_forward_ref(q, k, v, w, b, g, scale, h0, cfg: OracleCfg):
    """Forward in kernel semantics (scores.py + solve.py + cd_slim.py) on head-major inputs:
    returns o, h_final and the residuals A, Aqk, h_pre_all, v_new_all (chunked)."""
    st = wy_stage_ref(q, k, v, w, b, g, scale, cfg)
    if h0 is None:
        h0 = q.new_zeros(q.shape[:2] + (q.shape[-1], q.shape[-1]))
    o, hf, hp, vn = inter_chunk_scan_ref(st["Aqk"], st["wp"], st["u"], st["kg"], st["qg"],
                                         st["gc_last"], scale, h0, cfg, make_dot(cfg.dot_mode))
    return dict(o=from_chunks(o), h_final=hf, A=st["A"], Aqk=st["Aqk"], h_pre=hp, v_new=vn)


def grad_ref(q, k, v, w, b, g, scale, h0=None, cfg: OracleCfg = OracleCfg(), loss="sq"):
    """Gradient oracle: torch autograd of ``forward_ref`` (the analogue of
    ``jax.grad(forward_ref)`` in tests_gdn2/test_t5_grad_vs_reference.py:12-20).

    The loss is sum(o^2) + sum(h_final^2).  Inputs are head-major tensors of any float dtype;
    the computation runs in that dtype.  Returns dict o, h_final, dq, dk, dv, dw, db, dg, dh0.
    """
    leaves = [t.detach().clone().requires_grad_(True) for t in (q, k, v, w, b, g)]
    if h0 is None:
        h0 = q.new_zeros(q.shape[:2] + (q.shape[-1], q.shape[-1]))
    h0l = h0.detach().clone().requires_grad_(True)
    o, hf = forward_ref(*leaves, scale, h0l, cfg)
    L = (o * o).sum() + (hf * hf).sum()
    grads = torch.autograd.grad(L, leaves + [h0l])
    out = dict(o=o.detach(), h_final=hf.detach())
    for n, gr in zip(("dq", "dk", "dv", "dw", "db", "dg", "dh0"), grads):
        out[n] = gr
    return out


def rel_l2(a, b, floor=1e-8):
    """||a-b||_2 / ||b||_2 with an absolute floor (tests_gdn2/conftest.py:24-27)."""
    a = np.asarray(a.detach().cpu().double() if torch.is_tensor(a) else a, np.float64)
    b = np.asarray(b.detach().cpu().double() if torch.is_tensor(b) else b, np.float64)
    n, d = np.linalg.norm((a - b).ravel()), np.linalg.norm(b.ravel())
    return float(n if d < floor else n / d)


def canonical_flops(B, H, L, D, T=64):
    """Dense-convention FLOPs of one gradient evaluation: forward and backward."""
    n = B * H * L
    f = n * (10 * T * D + 6 * D * D)
    bwd = n * (22 * T * D + 12 * D * D + 4 * T * T)
    return f, bwd



