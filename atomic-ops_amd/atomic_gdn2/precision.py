"""Host-side numerics helpers (reference: atomic_gdn2/precision.py:41-52).

The matmul dot modes themselves (``highest`` / ``bf16x3`` / ``default``) live in the HIP
kernels; these torch helpers serve the host-side finishing step (``_fin``, ``sanitize``) and
callers that import the reference's precision module (``exp_nonpos``, ``exp_clipped``: the
kernels compute the same functions on the device, ``gdn2_common.hpp``).  The backward kernels
gate the derivative of exp(min(x, 0)) with 1{x <= 0}, the derivative autograd takes, not with
the mask returned here.
"""
import torch


def exp_nonpos(x):
    """exp(min(x,0)) and mask 1{x<0}.  The mask must not gate dgc contributions."""
    return torch.exp(torch.clamp(x, max=0.0)), (x < 0.0).to(x.dtype)


def exp_clipped(x, lo, hi):
    return torch.exp(torch.clamp(x, lo, hi)), ((x >= lo) & (x <= hi)).to(x.dtype)


def sanitize(x, clip: float):
    """clip to +-clip, NaN -> 0, +-inf -> +-clip."""
    return torch.nan_to_num(torch.clamp(x, -clip, clip), nan=0.0, posinf=clip, neginf=-clip)
