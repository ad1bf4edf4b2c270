"""GPU checks at the benchmark configurations' full sizes, and the failure path.

* config 3 at B4 H6 L4096 (two internal segments), B4 H2 L4096 and B4 H4 L2048: every output
  and gradient finite, one (batch, head) sequence against the float64 oracle run on it alone;
* config 4 at B8 H16 L32768 D128 with bf16 inputs as 8 calls of 4096 tokens (h0 = previous
  h_final): bit-equal to one call over the whole length, finite, one sequence against the
  float64 token recurrence;
* config 5, the benchmark LM at its real width (d_model 512, H 6, D 128, 8 blocks): one
  training step's loss and the gradients of the embedding and of one GDN-2 block against the
  same LM whose operator is the float64 oracle (batch 1, 256 tokens);
* NaN, +-Inf and huge inputs (the reference's clip plumbing test,
  tests/test_clip_config_plumbing.py:23-57): every output and gradient finite and within the
  configured clip, a tight and a loose clip give different results, and the poison stays
  where the recurrence carries it (other heads and earlier chunks bit-equal to a clean run).
"""
import math

import numpy as np
import pytest
import torch

from conftest import rel_l2
from test_gpu_parity import GATE, NAMES, banner, base_cfg, hip_grad, oracle_grad

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")


@pytest.mark.parametrize("H,L", [(6, 4096), (2, 4096), (4, 2048)])
def test_config3_cells_full_size(H, L):
    """Config 3's cells at their own shapes (B4 D128; L4096 is two internal segments; the grids
    of the scans, 8 H workgroups per batch row, and of the chunk-parallel kernels differ by
    cell): every output and gradient finite, one (batch, head) sequence against the float64
    oracle run on it alone."""
    from atomic_gdn2.synthetic import make_inputs_np
    banner(f"config3 B4 H{H} L{L} full size")
    arrs, scale = make_inputs_np(4, H, L, 128, seed=3)
    cfg = base_cfg()
    hip = hip_grad(cfg, scale, arrs)
    for n, t in hip.items():
        assert torch.isfinite(t).all(), n
    bi, hi = 2, H - 1
    ref = oracle_grad(cfg, scale, [a[bi:bi + 1, hi:hi + 1] for a in arrs])
    errs = {n: rel_l2(hip[n][bi:bi + 1, hi:hi + 1], ref[n]) for n in ("o", "h_final") + NAMES}
    banner(f"config3 H{H} L{L} slice {(bi, hi)} rel-L2 {errs}")
    assert max(errs.values()) <= GATE, errs


def test_config4_b8_h16_l32768_bf16_full_size():
    from atomic_gdn2 import make_blr_trainable
    from atomic_gdn2.synthetic import make_inputs_device
    from oracle import gdn2_oracle as O
    banner("config4 B8 H16 L32768 bf16, 8 calls of 4096")
    B, H, D, Lc, ncall = 8, 16, 128, 4096, 8
    xs, scale = make_inputs_device(B, H, Lc * ncall, D, seed=4, dtype=torch.bfloat16)
    fn = make_blr_trainable(base_cfg(), scale)
    outs, h = [], None
    with torch.no_grad():
        for c in range(ncall):
            o, h = fn(*(x[:, :, c * Lc:(c + 1) * Lc] for x in xs), h)
            outs.append(o)
        o_one, h_one = fn(*xs)
    torch.cuda.synchronize()
    o_calls = torch.cat(outs, dim=2)
    del outs
    assert torch.isfinite(o_calls).all() and torch.isfinite(h).all()
    assert torch.equal(o_calls, o_one) and torch.equal(h, h_one)
    bi, hi = 5, 11
    t = [x[bi:bi + 1, hi:hi + 1].double().cpu().transpose(1, 2) for x in xs]      # (1, L, 1, D)
    ro, rh = O.token_serial_ref(t[0], t[1], t[2], t[5], t[4], t[3], scale)
    eo = rel_l2(o_calls[bi:bi + 1, hi:hi + 1].transpose(1, 2), ro)
    eh = rel_l2(h[bi:bi + 1, hi:hi + 1], rh)
    banner(f"config4 slice {(bi, hi)} rel-L2 o {eo:.2e} h_final {eh:.2e}")
    assert eo <= GATE and eh <= GATE


def test_config5_full_width_lm_step_vs_oracle_operator():
    from atomic_gdn2 import e2e_lm
    from atomic_gdn2.e2e_lm import LM, LMConfig
    from oracle.gdn2_oracle import OracleCfg, forward_ref_blhd
    banner("config5 full-width LM (d_model 512, H6, D128, 8 blocks) vs oracle operator")
    cfg = LMConfig()
    op = e2e_lm.operator_cfg()
    torch.manual_seed(0)
    gpu = LM(cfg, e2e_lm.blhd_kernel(op, cfg.d_head)).cuda()
    ocfg = OracleCfg.from_cfg(op)

    def oracle_kernel(q, k, v, w, b, g):
        return forward_ref_blhd(q, k, v, w, b, g, 1.0 / math.sqrt(cfg.d_head), None, ocfg)[0]

    cpu = LM(cfg, oracle_kernel).double()
    cpu.load_state_dict({k: v.detach().double().cpu() for k, v in gpu.state_dict().items()})
    ids = torch.randint(0, cfg.vocab_size, (1, 256), generator=torch.Generator().manual_seed(1))
    prev = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        lg = e2e_lm.lm_loss(gpu, ids.cuda())
        lg.backward()
    finally:
        torch.backends.cuda.matmul.allow_tf32 = prev
    lc = e2e_lm.lm_loss(cpu, ids)
    lc.backward()
    banner(f"config5 loss hip {float(lg):.6f} oracle {float(lc):.6f}")
    assert abs(float(lg) - float(lc)) <= 1e-4 * abs(float(lc))
    checked = 0
    for (name, pg), (_, pc) in zip(gpu.named_parameters(), cpu.named_parameters()):
        if not (name.startswith("embed") or ".3." in name):
            continue
        rel = rel_l2(pg.grad, pc.grad)
        assert rel <= GATE, (name, rel)
        checked += 1
    assert checked >= 8, checked


# ---------------------------------------------------------------- failure path
def _huge(B, H, L, D, seed):
    """tests/test_clip_config_plumbing.py:46-55: q, k, v ~ 30 N, w ~ 30 U(0.5, 1.5), b = 50, g = 0."""
    rng = np.random.default_rng(seed)
    sh = (B, H, L, D)
    q, k, v = (rng.normal(size=sh) * 30.0 for _ in range(3))
    w = rng.uniform(0.5, 1.5, size=sh) * 30.0
    b = np.full(sh, 50.0)
    g = np.zeros(sh)
    return [x.astype(np.float32) for x in (q, k, v, w, b, g)]


def _bounded(out, clip, tag):
    for n, t in out.items():
        assert torch.isfinite(t).all(), (tag, n)
        m = float(t.abs().max())
        assert m <= clip + 1.0, (tag, n, m, clip)


def test_huge_inputs_honour_tight_and_loose_clip():
    banner("huge inputs, clip 5e3 vs 1e4")
    arrs = _huge(1, 2, 128, 128, 1)
    tight = hip_grad(base_cfg(clip=5e3), 1.0, arrs)
    loose = hip_grad(base_cfg(clip=1e4), 1.0, arrs)
    _bounded(tight, 5e3, "tight")
    _bounded(loose, 1e4, "loose")
    # the raw values exceed both clips, so the configured clip must show in the result
    for n in ("o", "h_final"):
        mt, ml = float(tight[n].abs().max()), float(loose[n].abs().max())
        assert abs(mt - ml) > 1.0, (n, mt, ml)


@pytest.mark.parametrize("training", [True, False])
def test_nan_inf_poison_is_sanitized_and_contained(training):
    """NaN in q, +Inf in k, -Inf in g, 1e30 in v of sequence (0, 0), all at tokens >= 128.
    Outputs and gradients are finite and within clip; sequence (0, 1) and the first two chunks
    of (0, 0) equal a clean run bit for bit (the reference's sanitize points absorb the poison,
    precision.py:51-52).  Where the poison lands the values differ from the reference by design:
    its dense products spread a NaN through the zero triangles of A and the masks (0 * NaN),
    while the kernels skip those exact-zero blocks, so fewer entries are zeroed."""
    from atomic_gdn2 import make_blr_trainable
    from atomic_gdn2.synthetic import make_inputs_np
    banner(f"NaN / Inf / 1e30 poison, training={training}")
    arrs, scale = make_inputs_np(1, 2, 256, 128, seed=5)
    bad = [a.copy() for a in arrs]
    bad[0][0, 0, 140, 5] = np.nan                 # q
    bad[1][0, 0, 150, 7] = np.inf                 # k
    bad[5][0, 0, 200, 3] = -np.inf                # g
    bad[2][0, 0, 170, :] = 1e30                   # v
    cfg = base_cfg()
    if training:
        clean, pois = hip_grad(cfg, scale, arrs), hip_grad(cfg, scale, bad)
    else:
        fn = make_blr_trainable(cfg, scale)
        with torch.no_grad():
            run = lambda a: dict(zip(("o", "h_final"), fn(*(torch.from_numpy(x).cuda() for x in a))))
            clean, pois = run(arrs), run(bad)
        torch.cuda.synchronize()
    _bounded(pois, cfg.clip, "poisoned")
    for n in clean:
        assert torch.equal(clean[n][:, 1], pois[n][:, 1]), ("other head", n)
    assert torch.equal(clean["o"][:, 0, :128], pois["o"][:, 0, :128]), "earlier chunks"
