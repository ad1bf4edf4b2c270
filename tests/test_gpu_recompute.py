"""The selective-recompute backward (gdn2_desc.state_ckpt = K >= 1) against the stored form
(K = 0, the state entering every chunk kept, as in the reference's residual, pipeline.py:25).

The recomputed states are the forward scan's own update with the same operands in the same
MFMA order, so every output and gradient must equal the stored form's bit for bit, for any K
(a ragged last block, K above the chunk count) and both head sizes; and the checkpoints kept
in the residual must be exactly the stored states of chunks 0, K, 2K, ...
"""
import ctypes

import numpy as np
import pytest
import torch

from conftest import mk_inputs
from test_gpu_parity import GATE, NAMES, banner, base_cfg, compare, oracle_grad, to_dev

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")


def _grad(cfg, scale, arrs, h0, ckpt):
    from atomic_gdn2 import make_blr_trainable
    xs = [t.requires_grad_(True) for t in to_dev(arrs)]
    h0t = torch.from_numpy(h0).cuda().requires_grad_(True)
    o, hf = make_blr_trainable(cfg, scale, state_ckpt=ckpt)(*xs, h0t)
    gr = torch.autograd.grad((o * o).sum() + (hf * hf).sum(), xs + [h0t])
    torch.cuda.synchronize()
    out = dict(o=o.detach(), h_final=hf.detach())
    out.update(zip(NAMES + ("dh0",), gr))
    return out


@pytest.mark.parametrize("D", [64, 128])
def test_recompute_equals_stored_bitwise(D):
    banner(f"recompute vs stored states, D={D}, L=320 (5 chunks)")
    cfg = base_cfg()
    scale = D ** -0.5
    arrs = mk_inputs(2, 320, 2, D, 21, g=0.1, layout="bhld")
    h0 = (np.random.default_rng(22).normal(size=(2, 2, D, D)) * 0.1).astype(np.float32)
    ref = _grad(cfg, scale, arrs, h0, 0)
    for n, t in ref.items():
        assert torch.isfinite(t).all(), n
    for ck in (1, 2, 3, 4, 32):
        got = _grad(cfg, scale, arrs, h0, ck)
        diff = {n: float((got[n] - ref[n]).abs().max()) for n in ref if not torch.equal(got[n], ref[n])}
        assert not diff, (ck, diff)
    ora = oracle_grad(cfg, scale, arrs, h0)
    compare(got, ora, GATE, names=("o", "h_final") + NAMES + ("dh0",))


def test_recompute_xcd_grouped_order_bitwise():
    """With B*H a multiple of 8 the backward groups whole (batch, head)s per XCD and dispatches
    their full checkpoint blocks before the single-chunk ones: B2 H4 (8 sequences) at 5 and 8
    chunks with K = 3 (two single-chunk blocks each) equals the stored form bit for bit."""
    banner("recompute vs stored, 8 sequences (XCD-grouped block order)")
    cfg = base_cfg()
    for L in (320, 512):
        arrs = mk_inputs(2, L, 4, 128, 26, g=0.1, layout="bhld")
        h0 = (np.random.default_rng(27).normal(size=(2, 4, 128, 128)) * 0.1).astype(np.float32)
        ref = _grad(cfg, 128 ** -0.5, arrs, h0, 0)
        got = _grad(cfg, 128 ** -0.5, arrs, h0, 3)
        for n in ref:
            assert torch.equal(got[n], ref[n]), (L, n)


def test_recompute_other_dot_modes_and_segments():
    """bf16x3 products, lean diagonal, eps > 0, and L = 4096 as two segments: recompute equals
    stored bit for bit."""
    banner("recompute vs stored: bf16x3 / lean / eps / two segments")
    for kw, L in ((dict(dot_mode="bf16x3", solve_dot_mode="bf16x3", b3_dot_mode="bf16x3"), 256),
                  (dict(diag="lean", wy_eps=1e-3, b3_dot_mode="bf16x3"), 256),
                  (dict(), 4096)):
        cfg = base_cfg(**kw)
        arrs = mk_inputs(1, L, 2, 128, 23, g=0.05, layout="bhld")
        h0 = (np.random.default_rng(24).normal(size=(1, 2, 128, 128)) * 0.1).astype(np.float32)
        ref = _grad(cfg, 128 ** -0.5, arrs, h0, 0)
        got = _grad(cfg, 128 ** -0.5, arrs, h0, 4)
        for n in ref:
            assert torch.equal(got[n], ref[n]), (kw, L, n)


@pytest.mark.parametrize("L,keep", [(448, [0, 3, 6]), (512, [0, 3, 6, 7])],
                         ids=["7 chunks", "8 chunks"])
def test_checkpoints_are_the_stored_states(L, keep):
    """The residual of state_ckpt = 3 keeps FA(h_pre^T) of the first chunk of each checkpoint
    block only, equal to the stored form's h_pre of those chunks: blocks [0, 3), [3, 6), [6, 7)
    for 7 chunks; for 8 the two chunks left over become single-chunk blocks (checkpoints 6, 7)."""
    from atomic_gdn2 import _lib
    from atomic_gdn2.synthetic import make_inputs
    banner(f"checkpoint residual L={L}")
    B, H, D = 1, 2, 128
    nc = L // 64
    xs, scale = make_inputs(B, H, L, D, seed=25)
    lib = _lib.lib()
    res = {}
    for ck in (0, 3):
        desc = _lib.make_desc(base_cfg(), B, H, L, D, scale, state_ckpt=ck)
        offs, tot = _lib.residual_layout(desc)
        r = torch.zeros(tot, dtype=torch.uint8, device="cuda")
        ws = torch.empty(lib.gdn2_fwd_workspace_bytes(ctypes.byref(desc), 1), dtype=torch.uint8, device="cuda")
        o = torch.empty(B, H, L, D, device="cuda")
        hf = torch.empty(B, H, D, D, device="cuda")
        _lib.check(lib.gdn2_fwd(ctypes.byref(desc), *map(_lib.ptr, xs), None, _lib.ptr(o), _lib.ptr(hf),
                                _lib.ptr(r), _lib.ptr(ws), _lib.stream_handle()), "gdn2_fwd")
        torch.cuda.synchronize()
        nck = nc if ck == 0 else len(keep)
        hp = r[offs[2]:offs[2] + B * H * nck * D * D * 4].view(torch.float32)
        res[ck] = (_lib.decode_residual("h_pre", hp, B, H, nck, 64, D), o)
        if ck:
            assert offs[3] - offs[2] < B * H * (nck + 1) * D * D * 4      # len(keep) states, not nc
    stored, o0 = res[0]
    ckpts, o3 = res[3]
    assert torch.equal(ckpts, stored[:, :, keep])
    assert torch.equal(o3, o0)
