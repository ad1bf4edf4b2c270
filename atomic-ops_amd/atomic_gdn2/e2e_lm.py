"""Synthetic language-model training step around the GDN-2 operator (the reference's
end-to-end benchmark LM).

The architecture follows the reference's benchmark LM (notebook
``benchmarks/notebooks/all-paths-speed.ipynb``, cell 2, ``PAYLOAD['corrected_original_lm.py']``
L10-80): embedding -> n_layers x GDN2Block -> RMSNorm -> logits tied to the embedding.  Each
block: q / k / v projections, each through a causal depthwise conv (kernel d_conv) and SiLU;
v clipped to +-50; q, k L2-normalised over the head dimension; erase gate b = sigmoid, write
gate w = sigmoid; per-head decay g = -min(|exp(decay_a) * softplus(decay_proj(x))|, g_max)
broadcast over the head dimension; the operator with h0 = 0; RMSNorm of its output times
SiLU(out_gate(x)) -> out_proj (residual); RMSNorm -> SwiGLU MLP (residual).  The default
LMConfig has 34,873,952 parameters, as the reference asserts.

The training step follows ``PAYLOAD['candidate_e2e.py']`` L15-29: mean cross-entropy of the
next-token logits, ``clip_by_global_norm(1.0)`` then AdamW (lr 1e-3, weight decay 0.01, the
optax defaults b1 0.9, b2 0.999, eps 1e-8; decay applied to every parameter).  Inputs are
uniform tokens in [0, vocab).  Matmuls run in fp32 (the reference sets
``jax_default_matmul_precision='highest'``).

This module is the operator's caller, written with torch (no flax / optax in this image); the
operator itself is ``make_blr_trainable`` on the HIP kernels.
"""
from __future__ import annotations

import dataclasses as dc
import math

import torch
import torch.nn.functional as F
from torch import nn

from .config import make_cfg
from .pipeline import make_blr_trainable


@dc.dataclass(frozen=True)
class LMConfig:
    vocab_size: int = 256
    d_model: int = 512
    n_heads: int = 6
    d_head: int = 128
    n_layers: int = 8
    mlp_mult: int = 2
    d_conv: int = 4
    g_max: float = 160.0 / 128
    decay_init: float = 0.05

    @property
    def proj_dim(self):
        return self.n_heads * self.d_head


def operator_cfg(**kw):
    """Operator configuration of the LM: the profile of the reference's published speed runs,
    'no_damping' (all_paths_speed_worker.py / isolated E2E: ``c.paths(profile='no_damping')``,
    candidate_common.py ``paths``: bt 128, bs2 64, BTL diagonal, wy_eps = 0).  With wy_eps = 0 the
    chunked WY form equals the token recurrence for every chunk size, so this build's chunk of
    64 computes the same operator; only the rounding differs.  Every product is fp32
    ('highest'): the profile's bf16x3 solve / backward products exist to avoid the cost of
    full-precision products on the TPU; on MI355X fp32 MFMA is the native path, and it is at
    least as accurate."""
    base = dict(bt=64, bc=32, score_bs=64, bs2=32, mb=8, diag="btl", wy_eps=0.0, dot_mode="highest",
                solve_dot_mode="highest", b3_dot_mode="highest")
    base.update(kw)
    return make_cfg(**base)


def blhd_kernel(cfg, d_head):
    """The operator on (B, L, H, D) tensors with h0 = 0 (the reference's adapter,
    ``PAYLOAD['candidate_e2e.py']`` L7-11 and ``candidate_common.py`` L63-66)."""
    fn = make_blr_trainable(cfg, 1.0 / math.sqrt(d_head))

    def run(q, k, v, w, b, g):
        sw = lambda x: x.transpose(1, 2).contiguous()
        o, _ = fn(*(sw(x) for x in (q, k, v, w, b, g)))
        return o.transpose(1, 2)

    return run


def _lecun_normal_(w: torch.Tensor, fan_in: int):
    # flax's default Dense init: truncated normal (+-2 sd) with variance 1 / fan_in
    std = math.sqrt(1.0 / fan_in) / 0.87962566103423978
    nn.init.trunc_normal_(w, std=std, a=-2 * std, b=2 * std)


class Dense(nn.Module):
    """y = x W (+ b), W of shape (in, out) as in flax."""

    def __init__(self, d_in, d_out, bias):
        super().__init__()
        self.weight = nn.Parameter(torch.empty(d_in, d_out))
        self.bias = nn.Parameter(torch.zeros(d_out)) if bias else None
        _lecun_normal_(self.weight, d_in)

    def forward(self, x):
        y = x @ self.weight
        return y + self.bias if self.bias is not None else y


class RMSNorm(nn.Module):
    def __init__(self, dim, eps=1e-6):
        super().__init__()
        self.scale = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x):
        return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + self.eps) * self.scale


class CausalDepthwiseConv(nn.Module):
    """out[t, c] = sum_j x[t - (K-1) + j, c] w[c, j] + bias[c] (zero history before t = 0)."""

    def __init__(self, dim, k):
        super().__init__()
        self.weight = nn.Parameter(torch.randn(dim, k) * 0.02)
        self.bias = nn.Parameter(torch.zeros(dim))
        self.k = k

    def forward(self, x):                      # (B, L, C)
        # K shifted multiply-adds on the (B, L, C) layout: element-wise work that streams x
        # K times, instead of a grouped convolution with one group per channel
        K = self.k
        y = torch.addcmul(self.bias, x, self.weight[:, K - 1])
        for s in range(1, K):
            y = torch.addcmul(y, F.pad(x[:, :-s], (0, 0, s, 0)), self.weight[:, K - 1 - s])
        return y


class GDN2Block(nn.Module):
    def __init__(self, cfg: LMConfig, kernel_fn):
        super().__init__()
        d, p, H = cfg.d_model, cfg.proj_dim, cfg.n_heads
        self.cfg, self.kernel_fn = cfg, kernel_fn
        self.q_proj, self.k_proj, self.v_proj = Dense(d, p, False), Dense(d, p, False), Dense(d, p, False)
        self.q_conv, self.k_conv, self.v_conv = (CausalDepthwiseConv(p, cfg.d_conv) for _ in range(3))
        self.erase_gate, self.write_gate = Dense(d, p, True), Dense(d, p, True)
        self.decay_a = nn.Parameter(torch.full((H,), math.log(math.expm1(cfg.decay_init))))
        self.decay_proj = Dense(d, H, True)
        self.out_gate = Dense(d, p, False)
        self.mixer_out_norm = RMSNorm(p)
        self.out_proj = Dense(p, d, False)
        self.mlp_norm = RMSNorm(d)
        self.gate_proj, self.up_proj = Dense(d, cfg.mlp_mult * d, False), Dense(d, cfg.mlp_mult * d, False)
        self.down_proj = Dense(cfg.mlp_mult * d, d, False)

    def forward(self, x):
        cfg = self.cfg
        B, L, _ = x.shape
        H, D = cfg.n_heads, cfg.d_head
        eps = 1e-6
        q = F.silu(self.q_conv(self.q_proj(x))).reshape(B, L, H, D)
        k = F.silu(self.k_conv(self.k_proj(x))).reshape(B, L, H, D)
        v = F.silu(self.v_conv(self.v_proj(x))).reshape(B, L, H, D).clamp(-50.0, 50.0)
        q = q * torch.rsqrt((q * q).sum(-1, keepdim=True) + eps)
        k = k * torch.rsqrt((k * k).sum(-1, keepdim=True) + eps)
        beta = torch.sigmoid(self.erase_gate(x)).reshape(B, L, H, D)
        wg = torch.sigmoid(self.write_gate(x)).reshape(B, L, H, D)
        ldh = -torch.exp(self.decay_a.clamp(-20, 20)) * F.softplus(self.decay_proj(x))
        ld = torch.nan_to_num(ldh, nan=0.0, posinf=0.0, neginf=-20.0)
        g = (-ld.abs().clamp(max=cfg.g_max)).unsqueeze(-1).expand(B, L, H, D)
        o = self.kernel_fn(q, k, v, wg, beta, g).reshape(B, L, H * D)
        og = self.out_gate(x)
        x = x + self.out_proj(self.mixer_out_norm(o) * F.silu(og))
        h2 = self.mlp_norm(x)
        return x + self.down_proj(F.silu(self.gate_proj(h2)) * self.up_proj(h2))


class LM(nn.Module):
    def __init__(self, cfg: LMConfig, kernel_fn):
        super().__init__()
        self.cfg = cfg
        self.embed = nn.Parameter(torch.randn(cfg.vocab_size, cfg.d_model) / math.sqrt(cfg.d_model))
        self.blocks = nn.ModuleList(GDN2Block(cfg, kernel_fn) for _ in range(cfg.n_layers))
        self.final_norm = RMSNorm(cfg.d_model)

    def forward(self, ids):
        x = self.embed[ids]
        for blk in self.blocks:
            x = blk(x)
        return self.final_norm(x) @ self.embed.t()


def n_params(model: nn.Module) -> int:
    return sum(p.numel() for p in model.parameters())


def lm_loss(model, ids):
    logits = model(ids)
    V = logits.shape[-1]
    return F.cross_entropy(logits[:, :-1].reshape(-1, V), ids[:, 1:].reshape(-1))


def clip_by_global_norm_(grads, max_norm):
    """optax.clip_by_global_norm: every g *= max_norm / max(global_norm, max_norm), in place."""
    norm = torch.linalg.vector_norm(torch.stack([torch.linalg.vector_norm(x) for x in grads]))
    torch._foreach_mul_(grads, max_norm / torch.clamp(norm, min=max_norm))
    return norm


class TrainStep:
    """One optimisation step: loss and gradients, clip_by_global_norm(max_norm), AdamW."""

    def __init__(self, model, lr=1e-3, weight_decay=0.01, max_norm=1.0):
        self.model = model
        self.params = [p for p in model.parameters()]
        self.opt = torch.optim.AdamW(self.params, lr=lr, betas=(0.9, 0.999), eps=1e-8,
                                     weight_decay=weight_decay, foreach=True)
        self.max_norm = max_norm

    def __call__(self, ids):
        self.opt.zero_grad(set_to_none=True)
        loss = lm_loss(self.model, ids)
        loss.backward()
        clip_by_global_norm_([p.grad for p in self.params], self.max_norm)
        self.opt.step()
        return loss.detach()


def make_lm(cfg: LMConfig = LMConfig(), op_cfg=None, device="cuda", seed=0):
    """The LM on `device` with the HIP operator (random init, seeded)."""
    torch.manual_seed(seed)
    op = operator_cfg() if op_cfg is None else op_cfg
    return LM(cfg, blhd_kernel(op, cfg.d_head)).to(device)


def synthetic_tokens(cfg: LMConfig, batch=8, length=2048, seed=0, device="cuda"):
    gen = torch.Generator().manual_seed(seed)
    return torch.randint(0, cfg.vocab_size, (batch, length), generator=gen).to(device)
