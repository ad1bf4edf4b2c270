"""GPU parity of the HIP operator against the CPU oracle and the golden fixtures.

Bar: o, h_final and all six input gradients within rel-L2 <= 2e-3
of the float64 oracle (autograd of the chunked-WY reference), as whole tensors and per 64-token
chunk.  Where the kernels' own dot
modes are mirrored by the kernel-semantics oracle, a much tighter bar is also asserted.
Every call goes through atomic_gdn2 -> libgdn2_hip.so (C ABI, include/gdn2.h).
"""
import ctypes
import os
from pathlib import Path

import numpy as np
import pytest
import torch

from conftest import DOMAIN, mk_inputs, rel_l2

pytestmark = pytest.mark.gpu

GATE = 2e-3
GOLD = Path(__file__).resolve().parent / "golden"
NAMES = ("dq", "dk", "dv", "dw", "db", "dg")


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")


def banner(msg):
    print(f"[gpu-test] {msg}", flush=True)


def to_dev(arrs, dtype=torch.float32):
    return [torch.from_numpy(np.ascontiguousarray(a)).to("cuda", dtype) for a in arrs]


def hip_grad(cfg, scale, arrs, h0=None, dtype=torch.float32, loss_h=True):
    """Forward + backward through the HIP operator; loss sum(o^2) + sum(h_final^2)."""
    from atomic_gdn2 import make_blr_trainable
    xs = [t.requires_grad_(True) for t in to_dev(arrs, dtype)]
    h0t = None
    if h0 is not None:
        h0t = torch.from_numpy(h0).cuda().float().requires_grad_(True)
    o, hf = make_blr_trainable(cfg, scale)(*xs, h0t)
    loss = (o * o).sum() + ((hf * hf).sum() if loss_h else 0.0)
    grads = torch.autograd.grad(loss, xs + ([h0t] if h0t is not None else []))
    torch.cuda.synchronize()
    out = dict(o=o.detach(), h_final=hf.detach())
    for n, gr in zip(NAMES + ("dh0",), grads):
        out[n] = gr
    return out


def oracle_grad(cfg, scale, arrs, h0=None):
    from oracle import gdn2_oracle as O
    t = [torch.from_numpy(np.asarray(a, np.float64)) for a in arrs]
    h = None if h0 is None else torch.from_numpy(np.asarray(h0, np.float64))
    return O.grad_ref(*t, scale, h, O.OracleCfg.from_cfg(cfg))


def kernel_oracle(cfg, scale, arrs, h0=None):
    """Kernel-semantics oracle (two-level scores, dot modes emulated) in float64."""
    from oracle import gdn2_oracle as O
    oc = O.OracleCfg.from_cfg(cfg)
    t = [torch.from_numpy(np.asarray(a, np.float64)) for a in arrs]
    h = None if h0 is None else torch.from_numpy(np.asarray(h0, np.float64))
    kf = O.kernel_forward_ref(*t, scale, h, oc)
    ch = lambda x: O.to_chunks(x, oc.bt)
    bw = O.backward_mega_ref(*map(ch, t), kf["A"], kf["Aqk"], kf["h_pre"], kf["v_new"],
                             ch(2 * kf["o"]), 2 * kf["h_final"], scale, oc)
    out = dict(o=kf["o"], h_final=kf["h_final"], dh0=bw["dh0"])
    for n in NAMES:
        out[n] = O.from_chunks(bw[n])
    return out


def compare(hip, ref, tol, names=("o", "h_final") + NAMES):
    """rel-L2 within tol for every named tensor as a whole, and for each 64-token chunk of the
    (B,H,L,D) ones: an error confined to some chunks cannot hide behind another chunk's larger
    values (the whole-tensor norm of dg is dominated by the last chunk's)."""
    errs = {n: rel_l2(hip[n], ref[n]) for n in names}
    bad = {n: e for n, e in errs.items() if not e <= tol}
    assert not bad, f"rel-L2 above {tol}: {bad}; all: {errs}"
    for n in names:
        if n in ("o",) + NAMES and hip[n].dim() == 4 and hip[n].shape[2] % 64 == 0:
            for c in range(hip[n].shape[2] // 64):
                e = rel_l2(hip[n][:, :, 64 * c:64 * (c + 1)], ref[n][:, :, 64 * c:64 * (c + 1)])
                assert e <= tol, f"{n} chunk {c}: rel-L2 {e:.2e} above {tol}"
    return errs


def base_cfg(**kw):
    from atomic_gdn2 import make_cfg
    d = dict(bt=64, bc=32, score_bs=64, bs2=32, mb=8, wy_eps=0.0, dot_mode="highest",
             solve_dot_mode="highest", b3_dot_mode="highest")
    d.update(kw)
    return make_cfg(**d)


# ---------------------------------------------------------------- library / primitives
def test_library_is_the_in_tree_hip_build():
    from atomic_gdn2 import _lib
    L = _lib.lib()
    assert L.gdn2_abi_version() == 3
    repo = Path(__file__).resolve().parents[1]
    assert Path(L._name).resolve().is_relative_to(repo), L._name
    maps = Path("/proc/self/maps").read_text()
    assert str(Path(L._name).resolve()) in maps


@pytest.mark.parametrize("mode", ["highest", "bf16x3", "default"])
@pytest.mark.parametrize("shape", [(16, 16, 16), (64, 32, 128), (32, 64, 64)])
def test_mfma_tile_layout(mode, shape):
    from atomic_gdn2 import _lib
    from oracle import gdn2_oracle as O
    M, N, K = shape
    banner(f"gemm probe {mode} {shape}")
    g = torch.Generator().manual_seed(M * N + K)
    A = torch.randn(M, K, generator=g)
    B = torch.randn(K, N, generator=g)
    C = torch.empty(M, N, device="cuda")
    Ad, Bd = A.cuda(), B.cuda()
    _lib.check(_lib.lib().gdn2_debug_gemm(_lib.DOT_IDS[mode], _lib.ptr(Ad), _lib.ptr(Bd), _lib.ptr(C), M, N, K,
                                          _lib.stream_handle()), "gemm")
    torch.cuda.synchronize()
    ref = O.make_dot(mode)(A.double(), B.double())
    assert rel_l2(C, ref) < 1e-6


def test_mfma_probe_does_the_products_it_counts():
    """The MFMA rate probe's lanes each end with the closed-form sum of their accumulators
    (eight accumulators of four elements, each 16 * iters for all-ones operands: 512 * iters),
    so the FLOPs the bench divides by were all issued; the guard past the end is untouched."""
    from atomic_gdn2 import _lib
    blocks, iters = 8, 64
    banner(f"mfma probe {blocks} x {iters}")
    out = torch.full((blocks * 256 + 256,), -7.0, device="cuda")
    _lib.check(_lib.lib().gdn2_debug_mfma(blocks, iters, _lib.ptr(out), _lib.stream_handle()), "mfma probe")
    torch.cuda.synchronize()
    assert bool((out[: blocks * 256] == 512.0 * iters).all()) and bool((out[blocks * 256:] == -7.0).all())


def test_stream_probe_copy_and_fill():
    """The HBM rate probe moves exactly the bytes it is given (copy) and writes its pattern
    (fill); the read mode leaves its sentinel target alone."""
    from atomic_gdn2 import _lib
    banner("stream probe 3 x 1 MiB")
    n = 1 << 20
    src = torch.randn(n // 4, device="cuda")
    dst = torch.full((n // 4 + 1024,), -7.0, device="cuda")        # 4 KB guard past the end
    L = _lib.lib()
    _lib.check(L.gdn2_debug_stream(0, _lib.ptr(src), _lib.ptr(dst), n, _lib.stream_handle()), "copy")
    torch.cuda.synchronize()
    assert torch.equal(dst[: n // 4], src) and bool((dst[n // 4:] == -7.0).all())
    _lib.check(L.gdn2_debug_stream(1, _lib.ptr(src), _lib.ptr(dst), n, _lib.stream_handle()), "read")
    torch.cuda.synchronize()
    assert torch.equal(dst[: n // 4], src)
    _lib.check(L.gdn2_debug_stream(2, None, _lib.ptr(dst), n, _lib.stream_handle()), "fill")
    torch.cuda.synchronize()
    i = torch.arange(n // 16, device="cuda")
    want = torch.stack([torch.ones_like(i, dtype=torch.float32), torch.full_like(i, 2, dtype=torch.float32),
                        torch.full_like(i, 3, dtype=torch.float32), (i & 255).float()], 1).reshape(-1)
    assert torch.equal(dst[: n // 4], want) and bool((dst[n // 4:] == -7.0).all())


# ---------------------------------------------------------------- config 1 (golden)
@pytest.fixture(scope="module")
def cfg1():
    from atomic_gdn2.synthetic import make_inputs_np, inputs_sha256
    arrs, scale = make_inputs_np(1, 2, 256, 128, seed=0)
    gold = np.load(GOLD / "config1_seed0.npz", allow_pickle=False)
    assert inputs_sha256(arrs) == str(gold["sha256"]), "synthetic generator drifted from the fixture"
    return arrs, scale, gold


def test_wy_stage_config1(cfg1):
    """Chunk-parallel stage outputs vs the kernel-semantics oracle and the fixture."""
    from atomic_gdn2 import _lib
    from oracle import gdn2_oracle as O
    arrs, scale, gold = cfg1
    banner("wy stage config1")
    cfg = base_cfg()
    xs = to_dev(arrs)
    B, H, L, D = arrs[0].shape
    nc = L // 64
    tt = lambda *s: torch.empty(*s, device="cuda")
    out = dict(aqk=tt(B, H, nc, 64, 64), akk=tt(B, H, nc, 64, 64), A=tt(B, H, nc, 64, 64),
               wp=tt(B, H, nc, 64, D), u=tt(B, H, nc, 64, D), kg=tt(B, H, nc, 64, D),
               qg=tt(B, H, nc, 64, D), gl=tt(B, H, nc, D))
    desc = _lib.make_desc(cfg, B, H, L, D, scale)
    _lib.check(_lib.lib().gdn2_wy_stage(ctypes.byref(desc), *map(_lib.ptr, xs),
                                        *(_lib.ptr(out[n]) for n in ("aqk", "akk", "A", "wp", "u", "kg", "qg", "gl")),
                                        _lib.stream_handle()), "wy_stage")
    torch.cuda.synchronize()
    ref = O.wy_stage_ref(*[torch.from_numpy(a).double() for a in arrs], scale, O.OracleCfg.from_cfg(cfg))
    pairs = dict(aqk="Aqk", akk="Akk", A="A", wp="wp", u="u", kg="kg", qg="qg", gl="gc_last")
    errs = {n: rel_l2(out[n], ref[m]) for n, m in pairs.items()}
    assert max(errs.values()) < 1e-5, errs
    for n, g in (("akk", "akk00"), ("A", "A00"), ("wp", "wp00"), ("u", "u00")):
        assert rel_l2(out[n][0, 0, 0], gold[g]) < 1e-5, n
    # structure: Akk strictly lower, A unit lower triangular, Aqk lower incl. diagonal
    A = out["A"].cpu()
    assert torch.all(torch.triu(A, 1) == 0) and torch.all(torch.diagonal(A, dim1=-2, dim2=-1) == 1)
    assert torch.all(torch.triu(out["akk"].cpu()) == 0) and torch.all(torch.triu(out["aqk"].cpu(), 1) == 0)
    # (I + Akk) A = I
    I = torch.eye(64)
    M = I + out["akk"].cpu().double()
    assert float((M @ A.double() - I).abs().max()) < 1e-4


@pytest.mark.parametrize("diag,bs2,sbs", [("btl", 32, 64), ("btl", 16, 64), ("lean", 32, 64), ("btl", 8, 64),
                                          ("btl", 8, 16), ("lean", 8, 32)])
def test_build_scores_takes_gc(cfg1, diag, bs2, sbs):
    """stages.build_scores(q, k, b, gc, scale, cfg), the reference's Kernel A signature
    (fwd/scores.py:87-97): gc is the caller's in-chunk cumulative gate, used as given.  Against
    the kernel-semantics oracle on the same gc (float64), and equal to the scores of
    gdn2_wy_stage, which forms gc from g itself (same in-chunk cumsum up to its rounding).
    Passing the raw g where gc belongs gives different scores (the argument is gc, not g)."""
    from atomic_gdn2.stages import build_scores, wy_stage
    from oracle import gdn2_oracle as O
    arrs, scale, _ = cfg1
    banner(f"build_scores(gc) {diag} bs2={bs2} score_bs={sbs}")
    cfg = base_cfg().with_(diag=diag, bs2=bs2, score_bs=sbs)
    q, k, v, w, b, g = (torch.from_numpy(a) for a in arrs)
    ch = lambda t: O.to_chunks(t, 64)
    gc = torch.cumsum(ch(g), dim=-2)                                   # float32, the caller's
    aqk, akk = build_scores(*(x.cuda() for x in (ch(q), ch(k), ch(b), gc)), scale, cfg)
    ra, rk = O.btl_scores(*(x.double() for x in (ch(q), ch(k), ch(b), gc)), scale, O.OracleCfg.from_cfg(cfg))
    ea, ek = rel_l2(aqk, ra), rel_l2(akk, rk)
    banner(f"  vs oracle on the same gc: aqk {ea:.2e} akk {ek:.2e}")
    assert ea < 1e-5 and ek < 1e-5
    st = wy_stage(*(x.cuda() for x in (q, k, v, w, b, g)), scale, cfg)
    assert rel_l2(st["aqk"], aqk) < 1e-5 and rel_l2(st["akk"], akk) < 1e-5
    _, akk_g = build_scores(*(x.cuda() for x in (ch(q), ch(k), ch(b), ch(g))), scale, cfg)
    assert rel_l2(akk_g, akk) > 1e-3


@pytest.mark.parametrize("kw", [dict(), dict(bs2=8), dict(score_bs=16, bs2=8)],
                         ids=lambda kw: ",".join(f"{k}={v}" for k, v in kw.items()) or "base")
def test_forward_residuals_config1(cfg1, kw):
    """gdn2_fwd through the C ABI: every residual sub-buffer and o / h_final per chunk vs
    the kernel-semantics oracle (localises a forward error to a stage and a chunk)."""
    from atomic_gdn2 import _lib
    from oracle import gdn2_oracle as O
    arrs, scale, _ = cfg1
    banner(f"fwd residuals config1 {kw}")
    cfg = base_cfg(**kw)
    xs = to_dev(arrs)
    B, H, L, D = arrs[0].shape
    nc = L // 64
    desc = _lib.make_desc(cfg, B, H, L, D, scale)
    offs, tot = _lib.residual_layout(desc)
    # residual and outputs start as NaN (all bits set), so an element the kernels leave unwritten shows
    res = torch.full((tot,), 255, dtype=torch.uint8, device="cuda")
    ws = torch.zeros(_lib.lib().gdn2_fwd_workspace_bytes(ctypes.byref(desc), 1), dtype=torch.uint8, device="cuda")
    o = torch.full((B, H, L, D), float("nan"), device="cuda")
    hf = torch.full((B, H, D, D), float("nan"), device="cuda")
    h0 = torch.zeros(B, H, D, D, device="cuda")
    _lib.check(_lib.lib().gdn2_fwd(ctypes.byref(desc), *map(_lib.ptr, xs), _lib.ptr(h0), _lib.ptr(o), _lib.ptr(hf),
                                   _lib.ptr(res), _lib.ptr(ws), _lib.stream_handle()), "gdn2_fwd")
    torch.cuda.synchronize()
    got = {}
    ends = list(offs[1:]) + [tot]
    for n, off, end in zip(_lib.RES_NAMES, offs, ends):
        flat = res[off:end].view(torch.float32).cpu()
        got[n.rstrip("T")] = _lib.decode_residual(n, flat, B, H, nc, 64, D)
    t = [torch.from_numpy(a).double() for a in arrs]
    oc = O.OracleCfg.from_cfg(cfg)
    st = O.wy_stage_ref(*t, scale, oc)
    kf = O.kernel_forward_ref(*t, scale, None, oc)
    ref = dict(aqk=st["Aqk"], A=st["A"], wp=st["wp"], kg=st["kg"], qg=st["qg"], gl=st["gc_last"],
               h_pre=kf["h_pre"], v_new=kf["v_new"])
    errs = {n: [rel_l2(got[n][:, :, c], ref[n][:, :, c]) for c in range(nc)] for n in ref}
    oc_ = O.to_chunks(o.cpu(), 64)
    ro = O.to_chunks(kf["o"], 64)
    errs["o"] = [rel_l2(oc_[:, :, c], ro[:, :, c]) for c in range(nc)]
    errs["h_final"] = [rel_l2(hf, kf["h_final"])]
    banner("per-chunk rel-L2: " + "; ".join(f"{n}: " + ",".join(f"{e:.1e}" for e in v) for n, v in errs.items()))
    # error map of o, chunk 0, head 0: rows in 16-row tiles x columns in 16-column slices
    d0 = (oc_[0, 0, 0] - ro[0, 0, 0]).abs()
    emap = d0.reshape(4, 16, D // 16, 16).amax(dim=(1, 3))
    banner("o chunk0 max-abs error by (row tile, col slice):\n" + "\n".join(
        " ".join(f"{x:.1e}" for x in row) for row in emap.tolist()))
    d1 = (got["h_pre"][0, 0, 1] - ref["h_pre"][0, 0, 1]).abs()
    emap = d1.reshape(D // 16, 16, D // 16, 16).amax(dim=(1, 3))
    banner("h after chunk0 max-abs error by (row tile, col slice):\n" + "\n".join(
        " ".join(f"{x:.1e}" for x in row) for row in emap.tolist()))
    banner("o chunk0 per-row max-abs error: " + " ".join(f"{x:.0e}" for x in d0.amax(dim=1).tolist()))
    banner("h after chunk0 per-row max-abs error: " + " ".join(f"{x:.0e}" for x in d1.amax(dim=1).tolist()))
    banner("h after chunk0 per-col max-abs error: " + " ".join(f"{x:.0e}" for x in d1.amax(dim=0).tolist()))
    bad = {n: v for n, v in errs.items() if max(v[1:] if n == "h_pre" else v) > 1e-5}
    assert not bad, bad


def test_forward_and_grads_config1(cfg1):
    arrs, scale, gold = cfg1
    banner("fwd+bwd config1")
    hip = hip_grad(base_cfg(), scale, arrs)
    errs = compare(hip, {n: gold[n] for n in ("o", "h_final") + NAMES}, GATE)
    ref = oracle_grad(base_cfg(), scale, arrs)
    tight = compare(hip, ref, 1e-4)
    banner(f"config1 rel-L2 vs fixture {errs}; vs live oracle max {max(tight.values()):.2e}")


# ---------------------------------------------------------------- reference test suite
@pytest.mark.parametrize("name,seed,g,k,b,dom", DOMAIN[:3] + [DOMAIN[3]])
def test_grad_vs_forward_ref(small_cfg, name, seed, g, k, b, dom):
    """tests_gdn2/test_t5_grad_vs_reference.py:23-30 (default dot modes, D=64, L=128)."""
    if name == "strong_decay":
        pytest.skip("reference underflows; covered by test_t2_domain")
    banner(f"T5 {name}")
    arrs = mk_inputs(1, 128, 1, 64, seed, g, k, b, layout="bhld")
    cfg = small_cfg.with_(g_max=1e3, bs2=32, wy_eps=0.0)
    hip = hip_grad(cfg, 1 / 8.0, arrs)
    compare(hip, oracle_grad(cfg, 1 / 8.0, arrs), 3e-3, NAMES)
    compare(hip, kernel_oracle(cfg, 1 / 8.0, arrs), 1e-4, NAMES)


@pytest.mark.parametrize("name,seed,g,k,b,dom", DOMAIN[4:])
def test_grad_other_domain_seeds(small_cfg, name, seed, g, k, b, dom):
    """The in-domain recipes of tests_gdn2/conftest.py:6-13 that T5 does not run (b close to 1,
    large stable k), through the HIP operator against the float64 oracle, at T5's size and gate,
    and against the kernel-semantics oracle at 1e-4."""
    banner(f"T5-style {name}")
    arrs = mk_inputs(1, 128, 1, 64, seed, g, k, b, layout="bhld")
    cfg = small_cfg.with_(g_max=1e3, bs2=32, wy_eps=0.0)
    hip = hip_grad(cfg, 1 / 8.0, arrs)
    compare(hip, oracle_grad(cfg, 1 / 8.0, arrs), 3e-3, ("o", "h_final") + NAMES)
    compare(hip, kernel_oracle(cfg, 1 / 8.0, arrs), 1e-4, NAMES)


@pytest.mark.parametrize("case", ["absorbed_tail", "planted_flat", "planted_flat_bt128", "planted_flat_bt256"])
def test_dg_on_flat_gate_segments(case):
    """dg where x = gc, gl - gc or gl is exactly 0 in fp32.  absorbed_tail: sequence (0, 1)
    of this seed has chunks whose last gates round away against gc, so gl - gc == 0 on a row
    whose true x is negative (with the strict mask 1{x < 0} of bwd/mega.py:47-48 its dg chunk
    missed the float64 gradient by 1.5e-3).  planted_flat: zero gates at the start of every
    64 tokens, tails of 1e-9 and of exact zeros, and a column zero over whole chunks; also at
    make_cfg()'s damped bt = 128 and at a damped bt = 256 (the kernels' 64-token parts).
    Every chunk of every gradient within 1e-4 of the float64 autograd oracle."""
    from atomic_gdn2 import make_cfg
    if case == "absorbed_tail":
        arrs = [np.ascontiguousarray(a[0:1, 1:2]) for a in mk_inputs(3, 2048, 6, 128, 903, g=0.05, layout="bhld")]
    else:
        arrs = list(mk_inputs(1, 512, 2, 128, 41, g=0.3, layout="bhld"))
        g = arrs[5].reshape(1, 2, 8, 64, 128).copy()
        g[..., 0:5, 0:4] = 0.0
        g[..., 40:64, 4:8] = -1e-9
        g[..., 48:64, 9:12] = 0.0
        g[..., :, 8] = 0.0
        arrs[5] = g.reshape(1, 2, 512, 128)
    banner(f"flat gate segments {case} {arrs[0].shape}")
    cfg = {"planted_flat_bt128": make_cfg(),
           "planted_flat_bt256": base_cfg(bt=256, bc=128, score_bs=128, bs2=32, mb=8, wy_eps=1e-3)}.get(case, base_cfg())
    hip = hip_grad(cfg, 128 ** -0.5, arrs)
    errs = compare(hip, oracle_grad(cfg, 128 ** -0.5, arrs), 1e-4)
    banner(f"flat gate segments {case}: max rel-L2 {max(errs.values()):.2e}")


def test_forward_matches_token_serial(small_cfg):
    from oracle import gdn2_oracle as O
    banner("T5 token serial")
    arrs = mk_inputs(1, 128, 1, 64, 0, layout="bhld")
    hip = hip_grad(small_cfg, 1 / 8.0, arrs)
    sw = lambda a: torch.from_numpy(np.swapaxes(a, 1, 2)).double()
    q, k, v, w, b, g = map(sw, arrs)
    ots, _ = O.token_serial_ref(q, k, v, g, b, w, 1 / 8.0)
    assert rel_l2(hip["o"].cpu().transpose(1, 2), ots) < 5e-3


@pytest.mark.parametrize("seed", [0, 1])
def test_directional_derivative_vs_token_serial_fd(seed):
    """T1 (tests_gdn2/test_t1_finite_diff.py:12-33) on the HIP operator: the derivative of
    sum(o^2) along a random direction in (q, k, v, b, g), from the kernels' VJP, against a
    central finite difference (eps 1e-5) of the float64 token recurrence, which shares no
    formula with the chunked WY form.  D = 64, L = 128."""
    from oracle import gdn2_oracle as O
    banner(f"T1 directional derivative, seed {seed}")
    D, L, H = 64, 128, 2
    scale = D ** -0.5
    arrs = mk_inputs(1, L, H, D, 40 + seed, layout="bhld")         # (B,H,L,D): q, k, v, w, b, g
    hip = hip_grad(base_cfg(), scale, arrs, loss_h=False)
    rng = np.random.default_rng(50 + seed)
    idx = {"dq": 0, "dk": 1, "dv": 2, "db": 4, "dg": 5}
    dirs = {n: torch.from_numpy(rng.normal(size=arrs[0].shape)) for n in idx}
    dd_hip = sum(float((hip[n].double().cpu() * dirs[n]).sum()) for n in idx)

    def f(theta):
        xs = [torch.from_numpy(np.asarray(a, np.float64)) for a in arrs]
        for n, i in idx.items():
            xs[i] = xs[i] + theta * dirs[n]
        q, k, v, w, b, g = (x.transpose(1, 2) for x in xs)          # (B,L,H,D)
        o, _ = O.token_serial_ref(q, k, v, g, b, w, scale)
        return float((o * o).sum())

    eps = 1e-5
    fd = (f(eps) - f(-eps)) / (2 * eps)
    assert abs(dd_hip - fd) / abs(fd) < 5e-3, (dd_hip, fd)


def test_causality_dq(small_cfg):
    """tests_gdn2/test_t5_grad_vs_reference.py:41-48: exact invariance of the prefix."""
    from atomic_gdn2 import make_blr_trainable
    banner("T5 causality")
    arrs = mk_inputs(1, 128, 1, 64, 0, g=0.05, layout="bhld")
    q, k, v, w, b, g = to_dev(arrs)
    fn = make_blr_trainable(small_cfg, 1 / 8.0)

    def dq_of(g_):
        qq = q.clone().requires_grad_(True)
        o, _ = fn(qq, k, v, w, b, g_)
        return torch.autograd.grad((o * o).sum(), qq)[0]

    p = 128 * 3 // 4
    g2 = g.clone()
    g2[:, :, p] -= 1.0
    assert float((dq_of(g)[:, :, :p] - dq_of(g2)[:, :, :p]).abs().max()) == 0.0


def test_determinism_and_dtype(small_cfg):
    """tests_gdn2/test_t5_grad_vs_reference.py:51-59."""
    banner("T5 determinism / dtype")
    arrs = mk_inputs(1, 128, 1, 64, 0, layout="bhld")
    g1 = hip_grad(small_cfg, 1 / 8.0, arrs)
    g2 = hip_grad(small_cfg, 1 / 8.0, arrs)
    assert all(torch.equal(g1[n], g2[n]) for n in NAMES + ("o", "h_final"))
    gb = hip_grad(small_cfg, 1 / 8.0, arrs, dtype=torch.bfloat16)
    assert all(gb[n].dtype == torch.bfloat16 for n in NAMES)
    assert gb["o"].dtype == torch.float32 and gb["h_final"].dtype == torch.float32


def test_segmented_equals_full():
    """tests_gdn2/test_segmentation.py:6-14."""
    from atomic_gdn2 import make_cfg
    banner("segmentation")
    cfg = make_cfg(bt=64, bc=32, score_bs=64, bs2=32, mb=8)
    arrs = mk_inputs(1, 256, 1, 64, 0, layout="bhld")
    a = hip_grad(cfg, 0.125, arrs, loss_h=False)
    b = hip_grad(cfg.with_(max_chunks_per_call=1), 0.125, arrs, loss_h=False)
    assert float((a["o"] - b["o"]).abs().max()) < 1e-5
    assert float((a["h_final"] - b["h_final"]).abs().max()) < 1e-5
    assert all(float((a[n] - b[n]).abs().max()) < 1e-4 for n in NAMES)


def test_b3_dot_mode_is_live(small_cfg):
    """tests_gdn2/test_t4_phantom_params.py:15-20."""
    banner("T4 b3 dot mode")
    arrs = mk_inputs(1, 128, 1, 64, 0, g=0.2, layout="bhld")
    base = hip_grad(small_cfg, 1 / 8.0, arrs)
    other = hip_grad(small_cfg.with_(b3_dot_mode="highest"), 1 / 8.0, arrs)
    assert max(float((base[n] - other[n]).abs().max()) for n in NAMES) > 1e-9


def test_bs2_changes_result_slightly(small_cfg):
    """tests_gdn2/test_t4_phantom_params.py:22-25."""
    banner("T4 bs2")
    arrs = mk_inputs(1, 128, 1, 64, 0, g=0.2, layout="bhld")
    a = hip_grad(small_cfg.with_(bs2=32), 1 / 8.0, arrs)
    b = hip_grad(small_cfg.with_(bs2=16, g_max=10.0), 1 / 8.0, arrs)
    d = max(float((a[n] - b[n]).abs().max()) for n in NAMES)
    assert 0 < d < 1e-2


# ---------------------------------------------------------------- config sweep
SWEEP = [
    dict(),
    dict(bs2=16),
    dict(bs2=64),
    dict(score_bs=32, bs2=16),
    dict(score_bs=32, bs2=32, mb=4),
    dict(mb=16),
    dict(diag="lean"),
    dict(wy_eps=0.01),
    dict(dot_mode="bf16x3", solve_dot_mode="bf16x3", b3_dot_mode="bf16x3"),
    dict(solve_dot_mode="default", b3_dot_mode="default"),
]


@pytest.mark.parametrize("kw", SWEEP, ids=lambda kw: ",".join(f"{k}={v}" for k, v in kw.items()) or "base")
@pytest.mark.parametrize("D", [64, 128])
def test_config_sweep(kw, D):
    from atomic_gdn2.synthetic import make_inputs_np
    banner(f"sweep D={D} {kw}")
    arrs, scale = make_inputs_np(2, 2, 192, D, seed=3)
    rng = np.random.default_rng(1)
    h0 = (rng.normal(size=(2, 2, D, D)) * 0.1).astype(np.float32)
    cfg = base_cfg(**kw)
    hip = hip_grad(cfg, scale, arrs, h0=h0)
    names = ("o", "h_final") + NAMES + ("dh0",)
    if "default" not in kw.values():
        compare(hip, oracle_grad(cfg, scale, arrs, h0), GATE, names)
    compare(hip, kernel_oracle(cfg, scale, arrs, h0), 1e-4 if "default" not in kw.values() else 2e-3, names)


# ---------------------------------------------------------------- config 2, full size
def test_config2_full_size_slices():
    """(4,6,2048,128): every (batch, head) sequence is independent, so two of them are checked
    against the oracle run on that sequence alone; all outputs must be finite."""
    from atomic_gdn2.synthetic import make_inputs_np
    banner("config2 full size")
    arrs, scale = make_inputs_np(4, 6, 2048, 128, seed=1)
    cfg = base_cfg()
    hip = hip_grad(cfg, scale, arrs)
    for n, t in hip.items():
        assert torch.isfinite(t).all(), n
    for (bi, hi) in ((0, 0), (3, 5)):
        sl = [a[bi:bi + 1, hi:hi + 1] for a in arrs]
        ref = oracle_grad(cfg, scale, sl)
        sub = {n: hip[n][bi:bi + 1, hi:hi + 1] for n in ("o", "h_final") + NAMES}
        errs = compare(sub, ref, GATE)
        banner(f"config2 slice {(bi, hi)} max rel-L2 {max(errs.values()):.2e}")


def test_two_segments_l4096():
    """L=4096 runs as two internal segments with h carried; (b,h) slice vs the oracle."""
    from atomic_gdn2.synthetic import make_inputs_np
    banner("L=4096 two segments")
    arrs, scale = make_inputs_np(1, 2, 4096, 128, seed=2)
    cfg = base_cfg()
    hip = hip_grad(cfg, scale, arrs)
    sl = [a[:, 1:2] for a in arrs]
    ref = oracle_grad(cfg, scale, sl)
    compare({n: hip[n][:, 1:2] for n in ("o", "h_final") + NAMES}, ref, GATE)


# ---------------------------------------------------------------- forward-only / bf16 inputs
def _fwd(cfg, scale, xs, h0=None):
    from atomic_gdn2 import make_blr_trainable
    with torch.no_grad():
        o, hf = make_blr_trainable(cfg, scale)(*xs, h0)
    torch.cuda.synchronize()
    return o, hf


def test_forward_only_equals_training_forward_bitwise():
    """The no-grad path (one kernel sequence over all L, no residual) equals the training path's
    segment loop bit for bit (segments of one chunk here)."""
    from atomic_gdn2 import make_blr_trainable
    banner("forward-only vs segmented training forward")
    cfg = base_cfg(max_chunks_per_call=1)
    arrs, scale = mk_inputs(1, 512, 2, 128, 3, layout="bhld"), 128 ** -0.5
    xs = [t.requires_grad_(True) for t in to_dev(arrs)]
    o1, h1 = make_blr_trainable(cfg, scale)(*xs)
    o2, h2 = _fwd(cfg, scale, [t.detach() for t in xs])
    assert torch.equal(o1.detach(), o2) and torch.equal(h1.detach(), h2)


@pytest.mark.parametrize("D", [64, 128])
def test_forward_only_odd_chunks_with_h0(D):
    """Without a residual the state scan computes o itself (output waves beside the chain);
    with one it leaves o to the chunk-parallel output kernel.  An odd chunk count (L=192, the
    scan's tail step) and a nonzero h0: both paths equal bit for bit, and within 2e-3 of the
    float64 oracle."""
    from atomic_gdn2 import make_blr_trainable
    from oracle import gdn2_oracle as O
    banner(f"forward-only odd chunks D={D}")
    cfg = base_cfg()
    scale = D ** -0.5
    arrs = mk_inputs(2, 192, 2, D, 8, layout="bhld")
    h0 = torch.randn(2, 2, D, D, device="cuda", generator=torch.Generator("cuda").manual_seed(9)) * 0.1
    xs = [t.requires_grad_(True) for t in to_dev(arrs)]
    o1, h1 = make_blr_trainable(cfg, scale)(*xs, h0)
    o2, h2 = _fwd(cfg, scale, [t.detach() for t in xs], h0)
    assert torch.equal(o1.detach(), o2) and torch.equal(h1.detach(), h2)
    t = [torch.from_numpy(a).double() for a in arrs]
    ro, rh = O.forward_ref(*t, scale, h0.double().cpu(), O.OracleCfg.from_cfg(cfg))
    assert rel_l2(o2, ro) < GATE and rel_l2(h2, rh) < GATE


@pytest.mark.parametrize("D", [64, 128])
def test_bf16_inputs_forward(D):
    """bf16 inputs are widened on load: bit-equal to the fp32 path on the same (bf16-rounded)
    values, and within 2e-3 of the float64 oracle on those values."""
    from oracle import gdn2_oracle as O
    banner(f"bf16 forward D={D}")
    cfg = base_cfg()
    scale = D ** -0.5
    arrs = mk_inputs(2, 256, 2, D, 4, layout="bhld")
    xb = [t.to(torch.bfloat16) for t in to_dev(arrs)]
    h0 = torch.randn(2, 2, D, D, device="cuda", generator=torch.Generator("cuda").manual_seed(5)) * 0.1
    ob, hb = _fwd(cfg, scale, xb, h0)
    of, hf = _fwd(cfg, scale, [t.float() for t in xb], h0)
    assert ob.dtype == torch.float32 and hb.dtype == torch.float32
    assert torch.equal(ob, of) and torch.equal(hb, hf)
    t = [x.double().cpu() for x in xb]
    ro, rh = O.forward_ref(*t, scale, h0.double().cpu(), O.OracleCfg.from_cfg(cfg))
    assert rel_l2(ob, ro) < 2e-3 and rel_l2(hb, rh) < 2e-3


def test_long_context_calls_carry_state_bitwise():
    """Config-4 protocol in miniature: one sequence as 4 external bf16 calls with h0 = previous
    h_final equals a single call over the whole length, bit for bit."""
    banner("long-context external segmentation")
    cfg = base_cfg()
    scale = 128 ** -0.5
    arrs = mk_inputs(1, 1024, 2, 128, 6, layout="bhld")
    xb = [t.to(torch.bfloat16) for t in to_dev(arrs)]
    o_all, h_all = _fwd(cfg, scale, xb)
    h, outs = None, []
    for s in range(4):
        o, h = _fwd(cfg, scale, [t[:, :, 256 * s:256 * (s + 1)].contiguous() for t in xb], h)
        outs.append(o)
    assert torch.equal(torch.cat(outs, dim=2), o_all) and torch.equal(h, h_all)
