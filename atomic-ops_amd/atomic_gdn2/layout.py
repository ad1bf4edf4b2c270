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
