"""Head-major layout (B,H,L,D) <-> chunks (B,H,nc,bt,D): pure reshapes (reference layout.py:4-15)."""
import torch


def to_chunks_hm(t, nc, bt):
    b, h, L, d = t.shape
    assert L == nc * bt, f"L={L} != nc*bt={nc * bt}"
    return t.reshape(b, h, nc, bt, d)


def from_chunks_hm(t):
    b, h, nc, bt, d = t.shape
    return t.reshape(b, h, nc * bt, d)


def causal_masks(T, device=None):
    i = torch.arange(T, device=device)
    return ((i[:, None] >= i[None, :]).to(torch.float32),
            (i[:, None] > i[None, :]).to(torch.float32))


def from_frag(x, R, C):
    """Row-major (..., R, C) copy of tiles stored in the kernels' fragment layout.

    ``x`` has R*C trailing elements per tile (any leading shape).  Fragment layout: 16x16
    blocks in row-major block order; inside a block, element 4*l + e with l = r + 16*c holds
    M[16*bi + r][16*bj + 4*c + e] (the float4 one MFMA lane loads).  Declared in include/gdn2.h.
    """
    lead = x.shape[:-1] if x.shape[-1] == R * C else x.shape[:-2]
    t = x.reshape(*lead, R // 16, C // 16, 4, 16, 4)
    n = len(lead)
    return t.permute(*range(n), n, n + 3, n + 1, n + 2, n + 4).reshape(*lead, R, C)


def to_frag(m):
    """Inverse of :func:`from_frag`: (..., R, C) -> (..., R*C) in fragment order."""
    *lead, R, C = m.shape
    n = len(lead)
    t = m.reshape(*lead, R // 16, 16, C // 16, 4, 4)          # bi, r, bj, c, e
    return t.permute(*range(n), n, n + 2, n + 3, n + 1, n + 4).reshape(*lead, R * C)
