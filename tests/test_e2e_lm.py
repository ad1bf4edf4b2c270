"""The end-to-end synthetic LM around the operator (reference benchmark LM,
notebook all-paths-speed.ipynb PAYLOAD['corrected_original_lm.py'] L10-80 and
PAYLOAD['candidate_e2e.py'] L7-29).

CPU: the architecture's parameter count (34,873,952, asserted by the reference), the causal
depthwise conv, the global-norm clip.  GPU: the LM's loss and every parameter gradient with the
HIP operator against the same LM whose operator is the float64 oracle, and a few AdamW steps.
"""
import math

import numpy as np
import pytest
import torch

from atomic_gdn2 import e2e_lm
from atomic_gdn2.e2e_lm import LM, LMConfig, CausalDepthwiseConv, clip_by_global_norm_, n_params


def passthrough(q, k, v, w, b, g):
    return v * w


def test_param_count_matches_reference():
    # candidate_e2e.py: assert count == 34873952 on the default LMConfig
    assert n_params(LM(LMConfig(), passthrough)) == 34_873_952


def test_causal_conv_matches_loop():
    torch.manual_seed(0)
    conv = CausalDepthwiseConv(5, 4).double()
    with torch.no_grad():
        conv.bias.copy_(torch.randn(5))
    x = torch.randn(2, 9, 5, dtype=torch.float64)
    y = conv(x)
    ref = torch.zeros_like(y)
    for t in range(9):
        for j in range(4):
            s = t - 3 + j
            if s >= 0:
                ref[:, t] += x[:, s] * conv.weight[:, j]
    ref += conv.bias
    assert torch.allclose(y, ref, atol=1e-12)


def test_clip_by_global_norm():
    g = [torch.full((3,), 2.0), torch.full((4,), 1.0)]
    n = clip_by_global_norm_(g, 1.0)
    assert math.isclose(float(n), math.sqrt(16.0), rel_tol=1e-6)
    assert torch.allclose(g[0], torch.full((3,), 0.5)) and torch.allclose(g[1], torch.full((4,), 0.25))
    small = [torch.full((2,), 0.1)]
    clip_by_global_norm_(small, 1.0)
    assert torch.allclose(small[0], torch.full((2,), 0.1))


def test_forward_shapes_and_loss_cpu():
    cfg = LMConfig(vocab_size=16, d_model=8, n_heads=2, d_head=4, n_layers=2)
    m = LM(cfg, passthrough)
    ids = torch.randint(0, 16, (2, 12))
    assert m(ids).shape == (2, 12, 16)
    loss = e2e_lm.lm_loss(m, ids)
    loss = loss.detach()
    assert torch.isfinite(loss) and abs(float(loss) - math.log(16)) < 2.0


TINY = LMConfig(vocab_size=32, d_model=48, n_heads=2, d_head=64, n_layers=2, mlp_mult=2)


@pytest.mark.gpu
def test_lm_gradients_match_oracle_operator():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    import sys
    from pathlib import Path
    sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
    from oracle.gdn2_oracle import OracleCfg, forward_ref_blhd
    print("[gpu-test] e2e LM tiny grads vs oracle", flush=True)
    op = e2e_lm.operator_cfg(wy_eps=0.0, solve_dot_mode="highest", b3_dot_mode="highest")
    torch.manual_seed(0)
    gpu = LM(TINY, e2e_lm.blhd_kernel(op, TINY.d_head)).cuda()
    ocfg = OracleCfg.from_cfg(op)

    def oracle_kernel(q, k, v, w, b, g):
        return forward_ref_blhd(q, k, v, w, b, g, 1.0 / math.sqrt(TINY.d_head), None, ocfg)[0]

    cpu = LM(TINY, oracle_kernel).double()
    cpu.load_state_dict({k: v.detach().double().cpu() for k, v in gpu.state_dict().items()})
    ids = torch.randint(0, TINY.vocab_size, (2, 128), generator=torch.Generator().manual_seed(1))
    lg = e2e_lm.lm_loss(gpu, ids.cuda())
    lg.backward()
    lc = e2e_lm.lm_loss(cpu, ids)
    lc.backward()
    assert abs(float(lg) - float(lc)) <= 1e-4 * abs(float(lc))
    worst = 0.0
    for (name, pg), (_, pc) in zip(gpu.named_parameters(), cpu.named_parameters()):
        a, b = pg.grad.double().cpu(), pc.grad
        rel = float((a - b).norm() / max(float(b.norm()), 1e-12))
        worst = max(worst, rel)
        assert rel <= 2e-3, (name, rel)
    print(f"[gpu-test] worst parameter-gradient rel-L2 {worst:.2e}", flush=True)


@pytest.mark.gpu
def test_lm_adamw_steps_reduce_loss():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    print("[gpu-test] e2e LM AdamW steps", flush=True)
    cfg = LMConfig(vocab_size=64, d_model=64, n_heads=2, d_head=64, n_layers=2)
    model = e2e_lm.make_lm(cfg, seed=0)
    step = e2e_lm.TrainStep(model)
    ids = e2e_lm.synthetic_tokens(cfg, batch=2, length=256, seed=0)
    losses = [float(step(ids)) for _ in range(6)]
    assert all(np.isfinite(losses))
    assert losses[-1] < losses[0]
