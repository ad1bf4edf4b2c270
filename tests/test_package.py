"""CPU tests of the host side: config surface (tests_gdn2/test_t9_package.py), the C ABI
library (loads, exports every symbol declared in include/gdn2.h, validates descriptors,
reports layouts), and the Python boundary's argument checks.  No GPU compute."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]


def test_import_and_prod_preset():
    from atomic_gdn2 import make_cfg
    c = make_cfg()
    assert (c.bt, c.score_bs, c.bs2, c.mb, c.diag) == (128, 128, 32, 8, "btl")
    assert c.btl_half_span_limit < 88.0
    assert (c.dot_mode, c.solve_dot_mode, c.b3_dot_mode) == ("highest", "bf16x3", "bf16x3")


@pytest.mark.parametrize("bs2", [8, 16, 32, 64, 128])
def test_gmax_tied_to_bs2(bs2):
    from atomic_gdn2 import make_cfg
    assert make_cfg(bs2=bs2).btl_half_span_limit < 88.0


def test_bad_config_rejected():
    from atomic_gdn2 import BLRConfig
    for kw in (dict(bt=100), dict(bs2=48), dict(mb=6), dict(diag="x"), dict(b3_dot_mode="fp8"),
               dict(wy_eps=1.0)):
        with pytest.raises(ValueError):
            BLRConfig(**kw)


def test_with_and_properties():
    from atomic_gdn2 import make_cfg, PROD
    c = make_cfg(bt=64, bc=32, score_bs=64, bs2=32)
    assert c.with_(bs2=16).bs2 == 16 and c.n_sub == 1 and c.n_inner == 2
    assert PROD is make_cfg


def _header_functions():
    txt = (ROOT / "include" / "gdn2.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(gdn2_\w+)\s*\(", txt, re.M)))


def test_library_exports_every_header_symbol():
    from atomic_gdn2 import _lib
    L = _lib.lib()
    names = _header_functions()
    assert len(names) >= 10, names
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    assert L.gdn2_abi_version() == 3


def test_descriptor_struct_matches_header():
    from atomic_gdn2 import _lib
    assert ctypes.sizeof(_lib.Gdn2Desc) == 14 * 4 + 4 * 8
    assert _lib.Gdn2Desc.seq_ld.offset == 48 and _lib.Gdn2Desc.state_ckpt.offset == 52
    assert _lib.Gdn2Desc.scale.offset == 56


def _desc(**kw):
    from atomic_gdn2 import make_cfg, _lib
    cfg = make_cfg(bt=64, bc=32, score_bs=64, bs2=32, mb=8, wy_eps=0.0)
    shape = dict(B=4, H=6, L=2048, D=128)
    shape.update({k: v for k, v in kw.items() if k in shape})
    cfg = cfg.with_(**{k: v for k, v in kw.items() if k not in shape})
    return _lib.make_desc(cfg, shape["B"], shape["H"], shape["L"], shape["D"], 128 ** -0.5)


def test_residual_layout_and_workspaces():
    from atomic_gdn2 import _lib
    offs, tot = _lib.residual_layout(_desc())
    N = 4 * 6 * 32
    sizes = [N * 64 * 64 * 4, N * 64 * 64 * 4, N * 128 * 128 * 4] + [N * 64 * 128 * 4] * 4 + [N * 128 * 4]
    for i, (o, s) in enumerate(zip(offs, sizes)):
        assert o % 256 == 0
        nxt = offs[i + 1] if i + 1 < len(offs) else tot
        assert nxt - o >= s
    L = _lib.lib()
    d = _desc()
    # [U^T], without a residual also [Kg | Wp | Qg | Aqk | gl] (with one they are residuals;
    # h_pre / v_new never leave the scan)
    assert L.gdn2_fwd_workspace_bytes(ctypes.byref(d), 1) == N * 64 * 128 * 4
    assert L.gdn2_fwd_workspace_bytes(ctypes.byref(d), 0) == N * (4 * 64 * 128 + 64 * 64 + 128) * 4
    assert L.gdn2_bwd_workspace_bytes(ctypes.byref(d)) >= N * (4 * 64 * 128 + 128 * 128 + 128) * 4


@pytest.mark.parametrize("kw,msg", [
    (dict(bt=512, bc=256, score_bs=128), "bt in"),
    (dict(D=96), "D in"),
    (dict(bs2=4, g_max=40.0), "bs2 >= 8"),
    (dict(L=2000), "divisible"),
    (dict(L=0), "non-positive"),
    (dict(B=0), "non-positive"),
])
def test_descriptor_validation(kw, msg):
    from atomic_gdn2 import _lib
    with pytest.raises(ValueError, match=msg):
        _lib.residual_layout(_desc(**kw))


@pytest.mark.parametrize("bt,bs2", [(64, 8), (128, 8), (128, 128), (256, 128), (256, 256)])
def test_all_inner_block_sizes_accepted(bt, bs2):
    """Every bs2 the reference's config admits at the supported chunk sizes is accepted; a
    diagonal block wider than 64 tokens adds the anchor buffer (two rows of D floats per
    64-token part) to both workspaces."""
    from atomic_gdn2 import _lib
    d = _desc(bt=bt, bc=bt // 2, score_bs=bt, bs2=bs2, g_max=160.0 / bs2)
    _lib.residual_layout(d)
    L = _lib.lib()
    d0 = _desc(bt=bt, bc=bt // 2, score_bs=bt, bs2=min(bs2, 64), g_max=160.0 / bs2)
    extra = 4 * 6 * 32 * 2 * 128 * 4 if bs2 > 64 else 0
    for wr in (0, 1):
        assert L.gdn2_fwd_workspace_bytes(ctypes.byref(d), wr) == L.gdn2_fwd_workspace_bytes(ctypes.byref(d0), wr) + extra
    assert L.gdn2_bwd_workspace_bytes(ctypes.byref(d)) == L.gdn2_bwd_workspace_bytes(ctypes.byref(d0)) + extra


def test_state_checkpoint_residual_layout():
    """state_ckpt = K keeps one state per checkpoint block instead of nc: nc // K blocks of K,
    then the nc % K chunks left over as single-chunk blocks when they are at most two (K = 3, 5
    at nc = 32: two more), else as one block (K = 7: one of 4); negative K is rejected."""
    from atomic_gdn2 import _lib
    d0 = _desc()
    offs0, tot0 = _lib.residual_layout(d0)
    for K, nck in ((1, 32), (2, 16), (3, 12), (4, 8), (5, 8), (7, 5), (32, 1), (100, 1)):
        d = _desc()
        d.state_ckpt = K
        offs, tot = _lib.residual_layout(d)
        assert offs[3] - offs[2] == 4 * 6 * nck * 128 * 128 * 4
        assert tot0 - tot == 4 * 6 * (32 - nck) * 128 * 128 * 4
    d = _desc()
    d.state_ckpt = -1
    with pytest.raises(ValueError, match="state_ckpt"):
        _lib.residual_layout(d)


def test_segment_stride_validation():
    from atomic_gdn2 import _lib
    d = _desc(L=1024)
    d.seq_ld = 512
    with pytest.raises(ValueError, match="seq_ld"):
        _lib.residual_layout(d)
    d.seq_ld = 4096
    _lib.residual_layout(d)


def test_null_pointers_rejected_without_gpu_work():
    from atomic_gdn2 import _lib
    d = _desc()
    st = _lib.lib().gdn2_fwd(ctypes.byref(d), *([None] * 12))
    assert st == 1 and b"null" in _lib.lib().gdn2_last_error()


@pytest.mark.parametrize("mode,nbytes,src,dst,msg", [
    (3, 4096, 16, 16, b"mode"),
    (0, 0, 16, 16, b"multiple of 4096"),
    (0, 4095, 16, 16, b"multiple of 4096"),
    (0, 4096, None, 16, b"null"),
    (2, 4096, None, None, b"null"),
    (0, 4096, 16, 24, b"aligned"),
])
def test_stream_probe_arguments_rejected_without_gpu_work(mode, nbytes, src, dst, msg):
    from atomic_gdn2 import _lib
    st = _lib.lib().gdn2_debug_stream(mode, src, dst, nbytes, None)
    assert st == 1 and msg in _lib.lib().gdn2_last_error()


@pytest.mark.parametrize("blocks,iters,out,msg", [
    (0, 16, 16, b"blocks and iters"),
    ((1 << 20) + 1, 16, 16, b"blocks and iters"),
    (1, 0, 16, b"blocks and iters"),
    (1, 16, None, b"null"),
])
def test_mfma_probe_arguments_rejected_without_gpu_work(blocks, iters, out, msg):
    from atomic_gdn2 import _lib
    st = _lib.lib().gdn2_debug_mfma(blocks, iters, out, None)
    assert st == 1 and msg in _lib.lib().gdn2_last_error()


def test_python_boundary_errors():
    from atomic_gdn2 import make_cfg, make_blr_trainable
    cfg = make_cfg(bt=64, bc=32, score_bs=64, bs2=32)
    fn = make_blr_trainable(cfg, 0.125)
    x = torch.zeros(1, 1, 100, 64)
    with pytest.raises(ValueError, match="divisible"):
        fn(x, x, x, x, x, x)
    y = torch.zeros(1, 1, 128, 64)
    with pytest.raises(RuntimeError, match="ROCm device"):
        fn(y, y, y, y, y, y)
    with pytest.raises(ValueError, match="shape"):
        fn(y, y, y, y, y, torch.zeros(1, 1, 128, 32))


@pytest.mark.parametrize("shape", [(1, 1, 0, 64), (0, 2, 128, 64), (1, 0, 128, 64)])
def test_empty_inputs_rejected(shape):
    """An empty batch, head or sequence axis is a ValueError at the Python boundary, with or
    without gradients, before any device work (the C ABI's own check of such a descriptor is in
    test_descriptor_validation)."""
    from atomic_gdn2 import make_cfg, make_blr_trainable
    fn = make_blr_trainable(make_cfg(bt=64, bc=32, score_bs=64, bs2=32), 0.125)
    x = torch.zeros(shape)
    with pytest.raises(ValueError, match="empty input"):
        fn(x, x, x, x, x, x)
    xg = [torch.zeros(shape, requires_grad=True) for _ in range(6)]
    with pytest.raises(ValueError, match="empty input"):
        fn(*xg)


def test_synthetic_inputs_recipe():
    from atomic_gdn2.synthetic import make_inputs_np
    (q, k, v, w, b, g), scale = make_inputs_np(1, 2, 128, 64, seed=0)
    assert scale == pytest.approx(1 / 8)
    for x in (q, k, w):
        assert np.allclose(np.linalg.norm(x.astype(np.float64), axis=-1), 1, atol=1e-6)
    assert (b > 0).all() and (b < 1).all() and (g < 0).all()
    rng = np.random.Generator(np.random.PCG64(0))
    draws = [rng.standard_normal((1, 2, 128, 64)) for _ in range(3)]   # order q, k, v
    assert np.array_equal(v, draws[2].astype(np.float32))


def test_fragment_layout_roundtrip_and_definition():
    from atomic_gdn2.layout import from_frag, to_frag
    from atomic_gdn2 import _lib
    m = torch.randn(2, 3, 64, 128)
    f = to_frag(m)
    assert torch.equal(from_frag(f, 64, 128), m)
    off = lambda i, j, C: ((i // 16) * (C // 16) + j // 16) * 256 + 4 * ((i % 16) + 16 * ((j % 16) // 4)) + j % 4
    for i, j in [(0, 0), (5, 7), (17, 33), (63, 127), (40, 90)]:
        assert f[1, 2, off(i, j, 128)] == m[1, 2, i, j]
    # residual decoding: a fragment sub-buffer comes back as the named quantity, a transposed
    # one (v_new is stored as FRAG(v_new^T)) un-transposed
    B, H, nc, T, D = 1, 2, 3, 64, 128
    wp = torch.randn(B, H, nc, T, D)
    assert torch.equal(_lib.decode_residual("wp", to_frag(wp).reshape(-1), B, H, nc, T, D), wp)
    vn = torch.randn(B, H, nc, T, D)
    flat = to_frag(vn.transpose(-1, -2).contiguous()).reshape(-1)
    assert torch.equal(_lib.decode_residual("v_new", flat, B, H, nc, T, D), vn)


def test_golden_fixture_inputs_are_reproduced():
    from atomic_gdn2.synthetic import make_inputs_np, inputs_sha256
    gold = np.load(ROOT / "tests" / "golden" / "config1_seed0.npz", allow_pickle=False)
    arrs, _ = make_inputs_np(1, 2, 256, 128, seed=0)
    assert inputs_sha256(arrs) == str(gold["sha256"])


def test_golden_fixture_matches_oracle():
    """The committed fixture is what the oracle computes today (oracle drift check)."""
    from atomic_gdn2.synthetic import make_inputs_np
    from oracle import gdn2_oracle as O
    gold = np.load(ROOT / "tests" / "golden" / "config1_seed0.npz", allow_pickle=False)
    arrs, scale = make_inputs_np(1, 2, 256, 128, seed=0)
    t = [torch.from_numpy(a).double() for a in arrs]
    gr = O.grad_ref(*t, scale, None, O.OracleCfg(bt=64, score_bs=64, bs2=32, mb=8, wy_eps=0.0))
    for n in ("o", "h_final", "dq", "dk", "dv", "dw", "db", "dg"):
        assert O.rel_l2(gold[n], gr[n]) < 1e-6, n
