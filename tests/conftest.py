"""Shared test setup: import paths, the ``gpu`` marker, and the reference suite's fixtures
restated (tests_gdn2/conftest.py:6-33 of the reference)."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "atomic-ops_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

# name, seed, g_scale, k_scale, b_scale, in_domain   (tests_gdn2/conftest.py:6-10)
SEEDS = [
    ("benign0", 0, 0.05, 1.0, 0.5, True), ("benign1", 1, 0.05, 1.0, 0.5, True),
    ("strong_decay", 2, 3.0, 1.0, 0.5, True), ("near_zero", 3, 0.001, 1.0, 0.5, True),
    ("b_near_one", 5, 0.3, 1.0, 0.95, True), ("large_k_stable", 4, 0.3, 8.0, 0.02, True),
    ("large_kb_OOD", 4, 0.3, 8.0, 4.0, False)]
DOMAIN = [s for s in SEEDS if s[5]]


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")
    config.addinivalue_line("markers", "slow: long-running")


def mk_inputs(bsz, L, H, D, seed, g=0.05, k=1.0, b=0.5, layout="blhd"):
    """tests_gdn2/conftest.py:14-21: q,k,v ~ 0.1 N, w = 1, b ~ b*U(.5,1), g = -|N*g|.
    Returns float32 numpy arrays in (B,L,H,D) or, with layout='bhld', (B,H,L,D)."""
    rng = np.random.default_rng(seed)
    sh = (bsz, L, H, D)
    q = rng.normal(size=sh) * 0.1
    kk = rng.normal(size=sh) * 0.1 * k
    v = rng.normal(size=sh) * 0.1
    w = np.ones(sh)
    bb = b * rng.uniform(0.5, 1.0, size=sh)
    gg = -np.abs(rng.normal(size=sh) * g)
    out = tuple(x.astype(np.float32) for x in (q, kk, v, w, bb, gg))
    if layout == "bhld":
        out = tuple(np.ascontiguousarray(np.swapaxes(t, 1, 2)) for t in out)
    return out


def rel_l2(a, b, floor=1e-8):
    """tests_gdn2/conftest.py:24-27."""
    import torch
    f = lambda x: (x.detach().cpu().double().numpy() if torch.is_tensor(x) else np.asarray(x, np.float64))
    a, b = f(a), f(b)
    n, d = np.linalg.norm((a - b).ravel()), np.linalg.norm(b.ravel())
    return float(n if d < floor else n / d)


def gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture
def small_cfg():
    """tests_gdn2/conftest.py:30-33."""
    from atomic_gdn2 import make_cfg
    return make_cfg(bt=64, bc=32, score_bs=64, bs2=32, mb=8, max_chunks_per_call=32)
