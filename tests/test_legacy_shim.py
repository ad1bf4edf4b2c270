"""The legacy ``atomic_ops`` API over the HIP operator (reference atomic_ops/, its tests
tests/test_configs.py, test_imports.py, test_pallas.py restated).

CPU: presets, validation, sanitize, memory estimate, imports.  GPU: the legacy entry points in
(B, L, H, D) against the float64 token-serial recurrence (forward) and the oracle's autograd
(gradients), and the legacy shape test.
"""
import numpy as np
import pytest
import torch

import atomic_ops
from atomic_ops.configs import (KAGGLE_LARGE, KAGGLE_MEDIUM, KAGGLE_SMALL, DEFAULT_CONFIG, KernelConfig,
                                clip_acc, sanitize, validate_inputs)
from conftest import rel_l2


def test_imports_and_version():
    from atomic_ops import (gdn2_forward_trainable, gdn2_forward, gdn2_pallas_forward_trainable,
                            KernelConfig, is_tpu_available, estimate_memory)
    assert gdn2_forward_trainable is not None and hasattr(atomic_ops, "__version__")
    assert is_tpu_available() is False


def test_default_config_is_medium():
    assert DEFAULT_CONFIG == KAGGLE_MEDIUM


def test_sanitize_removes_nan_and_clips():
    x = torch.tensor([float("nan"), float("inf"), -float("inf"), 5.0, 1e9])
    out = sanitize(x, KAGGLE_SMALL)
    assert bool(torch.all(torch.isfinite(out)))
    assert float(out[3]) == 5.0 and float(out[4]) == KAGGLE_SMALL.clip
    y = torch.tensor([2e5, -2e5, 1.0])
    assert torch.equal(clip_acc(y, KAGGLE_LARGE), sanitize(y, KAGGLE_LARGE))


def test_presets_and_rejected_configs():
    for cfg in (KAGGLE_SMALL, KAGGLE_MEDIUM, KAGGLE_LARGE):
        assert cfg.bt % cfg.bc == 0 and cfg.bc % cfg.mb == 0 and cfg.n_sub == 2
    for kw in (dict(bt=100, bc=64), dict(bt=256, bc=64), dict(bt=128, bc=64, mb=48), dict(wy_eps=1.0)):
        with pytest.raises(ValueError):
            KernelConfig(**kw)


def test_validate_inputs():
    q = torch.ones(2, 256, 4, 128)
    with pytest.raises(ValueError):
        validate_inputs(q, torch.ones(2, 256, 4, 64), q, q, q, q, 0.1, None, KAGGLE_MEDIUM)
    with pytest.raises(ValueError, match="d_head=128"):
        qq = torch.ones(2, 256, 4, 64)
        validate_inputs(qq, qq, qq, qq, qq, qq, 0.1, None, KAGGLE_MEDIUM)
    with pytest.raises(ValueError, match="divisible"):
        q3 = torch.ones(1, 192, 1, 128)
        validate_inputs(q3, q3, q3, q3, q3, q3, 0.1, None, KAGGLE_MEDIUM)
    assert validate_inputs(q, q, q, q, q, q, 0.1, None, KAGGLE_MEDIUM) == (2, 256, 4, 128, 1)


def test_memory_estimate_and_recommendation():
    per_chunk = 256 * 256 * 3 + 256 * 128 * 7 + 128 * 128 * 2
    assert atomic_ops.estimate_memory(2, 512, 4) == 2 * 4 * 2 * per_chunk * 4 / 2 ** 20
    assert atomic_ops.get_recommended_config(1, 2048, 1) == KAGGLE_SMALL
    assert atomic_ops.get_recommended_config(64, 8192, 32) == KAGGLE_LARGE


@pytest.mark.gpu
@pytest.mark.parametrize("preset", ["KAGGLE_SMALL", "KAGGLE_MEDIUM", "KAGGLE_LARGE"])
def test_legacy_entry_points_match_oracle(preset):
    """The preset's own operator (chunk config.bt = 128 / 256 with its wy_eps and clip, as the
    reference's TPU path runs it) through the legacy entry points, against the float64 oracle
    at that chunk; the forward also against the token recurrence."""
    config = {"KAGGLE_SMALL": KAGGLE_SMALL, "KAGGLE_MEDIUM": KAGGLE_MEDIUM, "KAGGLE_LARGE": KAGGLE_LARGE}[preset]
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    import sys
    from pathlib import Path
    sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
    from oracle.gdn2_oracle import OracleCfg, grad_ref, token_serial_ref
    from conftest import mk_inputs
    print("[gpu-test] legacy atomic_ops vs oracle", flush=True)
    arrs = mk_inputs(1, 512, 2, 128, seed=3, g=0.05)               # (B, L, H, D)
    rng = np.random.default_rng(7)
    h0 = (rng.normal(size=(1, 2, 128, 128)) * 0.1).astype(np.float32)
    scale = 128 ** -0.5
    dev = [torch.from_numpy(a).cuda() for a in arrs]
    o, hf = atomic_ops.gdn2_forward(*dev, scale, h0=torch.from_numpy(h0).cuda(), config=config)
    assert o.shape == (1, 512, 2, 128) and hf.shape == (1, 2, 128, 128)
    t = [torch.from_numpy(a).double() for a in arrs]
    sw = lambda x: x.transpose(1, 2)
    q, k, v, w, b, g = (sw(x) for x in t)
    # the token recurrence takes (B, L, H, D) and the order (q, k, v, g, b, w)
    ro, rh = token_serial_ref(t[0], t[1], t[2], t[5], t[4], t[3], scale, torch.from_numpy(h0).double())
    assert rel_l2(o, ro) < 2e-3 and rel_l2(hf, rh) < 2e-3
    # gradients of sum(o^2) + sum(h_final^2) through the trainable entry point
    xs = [x.clone().requires_grad_(True) for x in dev]
    o2, hf2 = atomic_ops.gdn2_forward_trainable(*xs, scale, config=config)
    ((o2 * o2).sum() + (hf2 * hf2).sum()).backward()
    ref = grad_ref(q, k, v, w, b, g, scale, None,
                   OracleCfg(bt=config.bt, score_bs=config.bt, bs2=64, mb=config.mb, wy_eps=config.wy_eps,
                             clip=config.clip, diag="lean", diff_clip=20.0))
    for x, n in zip(xs, ("dq", "dk", "dv", "dw", "db", "dg")):
        assert rel_l2(x.grad, sw(ref[n])) < 2e-3, n


@pytest.mark.gpu
@pytest.mark.parametrize("g_rate", [8.0, 30.0])
def test_legacy_strong_decay_beyond_the_btl_span(g_rate):
    """Gates far beyond BTL's span (|g| = 8 and 30 per token: half spans 128 and 480 over a
    32-token block, past the 88 at which the BTL legs overflow): the legacy operator forms every
    pair exactly with its decay clipped at e^-20 (atomic_ops/gdn2_fwd.py:60-65), and so does the
    shim (the exact diagonal over the whole 64-token chunk).  Forward against the float64 oracle
    with the same exact scores; the BTL operator on the same inputs does not match it."""
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    import sys
    from pathlib import Path
    sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
    from atomic_gdn2 import make_blr_trainable
    from atomic_ops.fallback import operator_cfg
    from oracle.gdn2_oracle import OracleCfg, forward_ref
    from conftest import mk_inputs
    print(f"[gpu-test] legacy strong decay g={g_rate}", flush=True)
    config = KernelConfig(bt=64, bc=32, mb=8, clip=1e4, wy_eps=0.0)
    arrs = mk_inputs(1, 256, 2, 128, seed=5, g=1.0)                 # (B, L, H, D)
    arrs = arrs[:5] + (np.full_like(arrs[5], -g_rate),)
    scale = 128 ** -0.5
    dev = [torch.from_numpy(a).cuda() for a in arrs]
    o, hf = atomic_ops.gdn2_forward(*dev, scale, config=config)
    sw = lambda x: x.transpose(1, 2)
    t = [sw(torch.from_numpy(a).double()) for a in arrs]
    oc = OracleCfg(bt=64, score_bs=64, bs2=64, mb=8, wy_eps=0.0, diag="lean", diff_clip=20.0)
    ro, rh = forward_ref(*t, scale, None, oc)
    eo, eh = rel_l2(sw(o), ro), rel_l2(hf, rh)
    print(f"[gpu-test]   rel-L2 o {eo:.2e} h_final {eh:.2e}", flush=True)
    assert torch.isfinite(o).all() and eo < 2e-3 and eh < 2e-3
    cb = operator_cfg(config).with_(diag="btl", bs2=32)
    with torch.no_grad():
        ob, _ = make_blr_trainable(cb, scale)(*(sw(x) for x in dev))
    assert rel_l2(ob, ro) > 1e-2


@pytest.mark.gpu
def test_legacy_pallas_shapes():
    # tests/test_pallas.py:15-41 (ones inputs; shapes only)
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    print("[gpu-test] legacy shapes", flush=True)
    shape = (2, 512, 4, 128)
    x = [torch.ones(shape, device="cuda", requires_grad=True) for _ in range(6)]
    out, h_final = atomic_ops.gdn2_pallas_forward_trainable(*x, 0.1)
    assert out.shape == shape and h_final.shape == (2, 4, 128, 128)
    out.sum().backward()
    assert all(t.grad is not None and bool(torch.isfinite(t.grad).all()) for t in x)
    out2, _ = atomic_ops.gdn2_pallas_forward(*(t.detach() for t in x), 0.1)
    assert out2.shape == shape


def test_operator_cfg_follows_the_reference_dispatch():
    """Every preset runs its own chunk (128, 256) with its wy_eps, as the reference's TPU path
    does; a chunk the kernels do not run would get the reference's off-TPU operator (wy_eps = 0,
    which is the same for every chunk size)."""
    from atomic_ops.fallback import operator_cfg
    for preset in (KAGGLE_SMALL, KAGGLE_MEDIUM, KAGGLE_LARGE):
        c = operator_cfg(preset)
        assert (c.bt, c.wy_eps, c.clip) == (preset.bt, preset.wy_eps, preset.clip)
        assert c.mb == min(preset.mb, preset.bt)
        # the legacy Kernel A's exact pairs (gdn2_fwd.py:60-65): the exact diagonal, clip 20
        assert (c.diag, c.bs2, c.diff_clip) == ("lean", 64, 20.0)
    c = operator_cfg(KernelConfig(bt=512, bc=256, mb=8, clip=1e4, wy_eps=1e-3))
    assert c.bt == 64 and c.wy_eps == 0.0
    c = operator_cfg(KernelConfig(bt=64, bc=32, mb=8, clip=1e4, wy_eps=1e-3))
    assert c.bt == 64 and c.wy_eps == 1e-3 and c.mb == 8
