"""Domain guards and the BTL canary (reference tests_gdn2/test_t2_domain.py and
test_t3_canary.py, restated).

CPU: the guard arithmetic (half span, preconditions, safe bs2, g clamp, bias init, I-2 stat).
GPU: the BTL validity boundary of the HIP scores against the exact (lean) diagonal with the
guard's recall (no silent failure, no false failure inside the domain), and the canary.
"""
import math

import numpy as np
import pytest
import torch

from atomic_gdn2 import make_cfg
from atomic_gdn2 import domain
from atomic_gdn2.config import BTL_STOP
from conftest import rel_l2

D, T = 64, 64


def test_half_span_of_constant_gate():
    # constant g = -c: gc[s] = -c (s+1), span of a bs2 block = c (bs2 - 1)
    for c, bs2 in ((0.5, 32), (2.0, 16), (6.0, 32)):
        gc = torch.cumsum(torch.full((1, 1, 2, T, D), -c), dim=-2)
        assert math.isclose(float(domain.half_span_max(gc, bs2)), 0.5 * c * (bs2 - 1), rel_tol=1e-5)
        g = torch.full((1, 1, 2 * T, D), -c)
        assert math.isclose(float(domain.half_span_from_g(g, T, bs2)), 0.5 * c * (bs2 - 1), rel_tol=1e-5)


def test_precondition_check_raises():
    # test_t2_domain.py:35-38
    g = -torch.full((1, 1, 128, 8), 6.0)
    with pytest.raises(RuntimeError):
        domain.check_preconditions(g, make_cfg(bs2=32, g_max=1e3), strict=True)
    r = domain.check_preconditions(g, make_cfg(bs2=32, g_max=1e3), strict=False)
    assert r["status"] == "STOP" and r["half_span_max"] > BTL_STOP
    assert domain.check_preconditions(-torch.full((1, 1, 128, 8), 0.1), make_cfg())["status"] == "ok"
    assert domain.check_preconditions(g, make_cfg(bs2=32, g_max=1e3, diag="lean"))["status"] == "ok"


def test_guard_helpers():
    assert domain.safe_bs2_for(1.25) == 64           # 1.25 * 128 / 2 = 80 is not < 80 -> next
    assert domain.safe_bs2_for(1.0) == 128
    assert domain.safe_bs2_for(5.0) == 16
    assert domain.safe_bs2_for(100.0) == 8
    t = torch.tensor([-0.5, -3.0, -10.0])
    assert torch.equal(domain.clamp_g(t, 2.0), torch.tensor([-0.5, -2.0, -2.0]))
    assert math.isclose(math.log1p(math.exp(domain.init_g_bias(0.05))), 0.05, rel_tol=1e-12)
    k = torch.ones(2, 3, 4)
    b = torch.full((2, 3, 4), 0.5)
    mx, mean = domain.bk2_stat(k, b)
    assert float(mx) == 2.0 and float(mean) == 2.0


def _akk(cfg, c):
    from atomic_gdn2.stages import build_scores
    rng = np.random.default_rng(0)
    q, k, b = (torch.from_numpy(rng.normal(size=(1, 1, 1, T, D)).astype(np.float32) * s).cuda()
               for s in (0.3, 0.3, 0.5))
    b = b.abs()
    g = torch.full((1, 1, 1, T, D), -c, device="cuda")
    gc = torch.cumsum(g, dim=-2)
    return build_scores(q, k, b, gc, 1 / 8.0, cfg)[1], gc


@pytest.mark.gpu
@pytest.mark.parametrize("c", [0.5, 1.0, 2.0, 2.5, 3.0, 4.0, 6.0, 8.0])
def test_btl_boundary_and_guard(c):
    # test_t2_domain.py:22-33
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    print(f"[gpu-test] T2 boundary c={c}", flush=True)
    bs2 = 32
    cb = make_cfg(bt=T, bc=32, score_bs=T, bs2=bs2, mb=8, diag="btl", g_max=1e3)
    Ab, gc = _akk(cb, c)
    Al, _ = _akk(cb.with_(diag="lean"), c)
    err = rel_l2(Ab, Al)
    hs = float(domain.half_span_max(gc, bs2))
    alarm = hs > BTL_STOP
    wrong = err > 1e-3
    assert not (wrong and not alarm), f"SILENT FAILURE c={c}: err={err:.2e} half_span={hs:.1f}"
    if hs < 60:
        assert not wrong, f"false failure inside domain: err={err:.2e}"


@pytest.mark.gpu
def test_canary_quiet_in_domain_and_fires_outside():
    # test_t3_canary.py:7-16
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    from atomic_gdn2.training.canary import btl_vs_lean_canary
    print("[gpu-test] T3 canary", flush=True)
    r = btl_vs_lean_canary(make_cfg(bt=64, bc=32, score_bs=64, bs2=32, mb=8), D=64, g_level=0.3)
    assert r["rel_err"] < 1e-4 and not r["alarm"]
    r = btl_vs_lean_canary(make_cfg(bt=64, bc=32, score_bs=64, bs2=32, mb=8, g_max=1e3), D=64, g_level=8.0)
    assert r["alarm"]
