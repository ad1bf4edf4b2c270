"""Random in-domain configurations against the float64 oracle: chunk 64 / 128 / 256, damping,
score and leaf blockings, checkpoint intervals 0-5, segment lengths, batch x head counts that
are and are not multiples of 8, D 64 / 128.  Outputs, the six gradients and dh0 of
sum(o^2) + sum(h_final^2) within rel-L2 2e-3, and every 64-token chunk of them within 1e-4
(measured at most ~6e-7).  The cases come from a fixed seed, so every run draws the same ones."""
import random

import numpy as np
import pytest
import torch

from conftest import mk_inputs, rel_l2
from test_gpu_parity import GATE, banner

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")


def _cases(n, seed=7):
    rnd = random.Random(seed)
    out = []
    while len(out) < n:
        bt = rnd.choice([64, 64, 128, 256])
        D = rnd.choice([64, 128])
        B, H = rnd.choice([1, 2, 3]), rnd.choice([1, 2, 3, 4, 5])
        if bt == 256:
            B, H = 1, rnd.choice([1, 2, 3])
        nch = rnd.randint(1, 6 if bt < 256 else 3)
        eps = rnd.choice([0.0, 1e-3, 0.02])
        ck = rnd.choice([0, 1, 2, 3, 4, 5])
        if bt > 64 and eps > 0 and ck == 0:
            ck = 3                          # damped big chunks need checkpoints (gdn2_desc)
        sbs = rnd.choice([s for s in (32, 64, 128, 256) if s <= bt and bt % s == 0])
        bs2 = rnd.choice([s for s in (16, 32, 64) if s <= sbs and sbs % s == 0])
        mb = rnd.choice([m for m in (4, 8, 16) if bt % m == 0 and (bt // m) & (bt // m - 1) == 0])
        kw = dict(bt=bt, bc=bt // 2, score_bs=sbs, bs2=bs2, mb=mb, wy_eps=eps,
                  max_chunks_per_call=rnd.choice([1, 2, 32]))
        out.append((B, H, bt * nch, D, kw, ck))
    return out


CASES = _cases(16)


@pytest.mark.parametrize("i", range(len(CASES)))
def test_random_config_matches_oracle(i):
    from atomic_gdn2 import make_cfg, make_blr_trainable
    from oracle import gdn2_oracle as O
    B, H, L, D, kw, ck = CASES[i]
    banner(f"random config {i}: B{B} H{H} L{L} D{D} {kw} state_ckpt {ck}")
    cfg = make_cfg(**kw, dot_mode="highest", solve_dot_mode="highest", b3_dot_mode="highest")
    scale = D ** -0.5
    arrs = mk_inputs(B, L, H, D, 300 + i, g=0.05, layout="bhld")
    h0 = (np.random.default_rng(400 + i).normal(size=(B, H, D, D)) * 0.1).astype(np.float32)
    xs = [torch.from_numpy(a).cuda().requires_grad_(True) for a in arrs]
    h0t = torch.from_numpy(h0).cuda().requires_grad_(True)
    o, hf = make_blr_trainable(cfg, scale, state_ckpt=ck)(*xs, h0t)
    grads = torch.autograd.grad((o * o).sum() + (hf * hf).sum(), xs + [h0t])
    torch.cuda.synchronize()
    got = dict(o=o.detach(), h_final=hf.detach())
    got.update(zip(("dq", "dk", "dv", "dw", "db", "dg", "dh0"), grads))
    t = [torch.from_numpy(np.asarray(a, np.float64)) for a in arrs]
    ref = O.grad_ref(*t, scale, torch.from_numpy(h0.astype(np.float64)), O.OracleCfg.from_cfg(cfg))
    errs = {n: rel_l2(got[n], ref[n]) for n in got}
    # and per 64-token chunk of every (B,H,L,D) tensor, where an error confined to some chunks
    # cannot hide behind another chunk's larger values (fp32 gives ~1e-6; the bar is 1e-4)
    per_chunk = {n: max(rel_l2(got[n][:, :, 64 * c:64 * (c + 1)], ref[n][:, :, 64 * c:64 * (c + 1)])
                        for c in range(L // 64))
                 for n in ("o", "dq", "dk", "dv", "dw", "db", "dg")}
    banner(f"random config {i}: max rel-L2 {max(errs.values()):.2e}, per chunk {max(per_chunk.values()):.2e}")
    assert max(errs.values()) < GATE, errs
    assert max(per_chunk.values()) < 1e-4, per_chunk
