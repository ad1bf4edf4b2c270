"""Pins for the CPU oracle (oracle/gdn2_oracle.py).  CPU only.

Each oracle function is checked against something that does not share its formula:
  * the reference's stored 80-digit Decimal known answers (D=4, L=256, 3 seeds, 2 objectives);
  * the token-serial recurrence (chunked WY == serial, any blocking, eps, h0);
  * brute-force O(T^2 D) scores; scipy's unit-lower triangular solve for the ladder inverse;
  * finite differences of the token-serial recurrence for the autograd gradients;
  * agreement of the analytic backward (kernel semantics, B1..B5) with autograd;
  * B4's closed form (b4_exact_f64_np) against autograd of the two-level scores.
Planted mistakes at the end show that each pin fails on a plausible slip.
"""
import json
import math
from pathlib import Path

import numpy as np
import pytest
import scipy.linalg
import torch

from oracle import gdn2_oracle as O

GOLD = Path(__file__).resolve().parent / "golden"


@pytest.fixture(autouse=True)
def _float64_default():
    """float64 default dtype for these tests only (collection of other modules is unaffected)."""
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    yield
    torch.set_default_dtype(prev)


def t64(x):
    return torch.as_tensor(np.asarray(x, np.float64))


def rand_inputs(B, H, L, D, seed, gscale=0.05, h0=False):
    rng = np.random.default_rng(seed)
    sh = (B, H, L, D)
    q = rng.normal(size=sh) * 0.3
    k = rng.normal(size=sh) * 0.3
    v = rng.normal(size=sh)
    w = rng.uniform(0.2, 1.0, size=sh)
    b = rng.uniform(0.2, 1.0, size=sh)
    g = -np.abs(rng.normal(size=sh)) * gscale
    out = [t64(x) for x in (q, k, v, w, b, g)]
    out.append(t64(rng.normal(size=(B, H, D, D)) * 0.1) if h0 else None)
    return out


def rel(a, b):
    return float(torch.linalg.norm((a - b).reshape(-1)) / max(float(torch.linalg.norm(b.reshape(-1))), 1e-300))


# ---------------------------------------------------------------- known answers
KAT = json.loads((GOLD / "kat_d4.json").read_text())


@pytest.mark.parametrize("seed", [0, 1, 2])
@pytest.mark.parametrize("alg", ["serial", "chunked"])
def test_decimal_known_answers(seed, alg):
    d = np.load(GOLD / f"kat_d4_seed{seed}.npz", allow_pickle=False)
    t = {k: t64(d[k]) for k in d.files}
    cfg = O.OracleCfg(bt=64, score_bs=64, bs2=32, mb=8, wy_eps=0.0)
    th = torch.zeros((), requires_grad=True)
    v = t["v"] + th * t["direction"]
    if alg == "serial":
        o, hf = O.token_serial_ref(t["q"], t["k"], v, t["g"], t["b"], t["w"], 0.5, t["h0"])
    else:
        o, hf = O.forward_ref_blhd(t["q"], t["k"], v, t["w"], t["b"], t["g"], 0.5, t["h0"], cfg)
    y = torch.cat([o.reshape(-1), hf.reshape(-1)])
    objs = {"natural": 0.5 * (y * y).sum(), "cancellation_stress": (t["coeff"] * y).sum()}
    for mode, f in objs.items():
        (gr,) = torch.autograd.grad(f, th, retain_graph=True)
        ref = KAT["cases"][f"{seed}/{mode}"]
        val_ref, grad_ref = float(ref["value"]), float(ref["gradient"])
        assert abs(float(f) - val_ref) <= 1e-12 * max(1.0, abs(val_ref)), (mode, float(f), val_ref)
        assert abs(float(gr) - grad_ref) <= 1e-12, (mode, float(gr), grad_ref)


# ---------------------------------------------------------------- chunked == serial
CFGS = [
    dict(),
    dict(bs2=16),
    dict(bs2=64),
    dict(score_bs=32, bs2=16),
    dict(score_bs=32, bs2=32, mb=4),
    dict(mb=16, wy_eps=0.05),
    dict(diag="lean"),
]


@pytest.mark.parametrize("kw", CFGS)
def test_chunked_equals_token_serial(kw):
    cfg = O.OracleCfg(**kw)
    q, k, v, w, b, g, h0 = rand_inputs(1, 2, 192, 16, 7, h0=True)
    o, hf = O.forward_ref(q, k, v, w, b, g, 0.25, h0, cfg)
    sw = lambda x: x.transpose(1, 2)
    if cfg.wy_eps == 0.0:
        os_, hs = O.token_serial_ref(sw(q), sw(k), sw(v), sw(g), sw(b), sw(w), 0.25, h0)
        assert rel(o, sw(os_)) < 1e-10 and rel(hf, hs) < 1e-10
    # kernel semantics (two-level scores, BTL or lean diagonal) agree with the oracle form
    kf = O.kernel_forward_ref(q, k, v, w, b, g, 0.25, h0, cfg)
    assert rel(kf["o"], o) < 1e-10 and rel(kf["h_final"], hf) < 1e-10


def test_damping_changes_result_consistently():
    """wy_eps > 0 is a different operator; both oracle forms must agree on it."""
    q, k, v, w, b, g, h0 = rand_inputs(1, 1, 128, 16, 3)
    c0, c1 = O.OracleCfg(), O.OracleCfg(wy_eps=0.1)
    o0, _ = O.forward_ref(q, k, v, w, b, g, 0.25, h0, c0)
    o1, _ = O.forward_ref(q, k, v, w, b, g, 0.25, h0, c1)
    assert rel(o1, o0) > 1e-4


# ---------------------------------------------------------------- scores
def brute_scores(q, k, b, gc, scale):
    """Triple loop over (i, j, d) in numpy float64 (tests/test_gdn2_full_math_correctness.py:169-183)."""
    q, k, b, gc = (np.asarray(x) for x in (q, k, b, gc))
    T, D = q.shape
    Aq = np.zeros((T, T)); Ak = np.zeros((T, T))
    for i in range(T):
        for j in range(i + 1):
            e = np.exp(gc[i] - gc[j])
            Aq[i, j] = scale * np.sum(q[i] * k[j] * e)
            if j < i:
                Ak[i, j] = np.sum(b[i] * k[i] * k[j] * e)
    return Aq, Ak


@pytest.mark.parametrize("kw", CFGS[:5] + [dict(diag="lean", bs2=16)])
def test_scores_brute_force(kw):
    cfg = O.OracleCfg(**kw)
    rng = np.random.default_rng(11)
    T, D = 64, 8
    q, k = rng.normal(size=(T, D)), rng.normal(size=(T, D))
    b = rng.uniform(0.2, 1, size=(T, D))
    gc = np.cumsum(-np.abs(rng.normal(size=(T, D))) * 0.2, axis=0)
    Aq_bf, Ak_bf = brute_scores(q, k, b, gc, 0.3)
    for fn in (O.blr_scores_ref, O.btl_scores):
        Aq, Ak = fn(t64(q), t64(k), t64(b), t64(gc), 0.3, cfg)
        assert np.max(np.abs(Aq.numpy() - Aq_bf)) < 1e-12
        assert np.max(np.abs(Ak.numpy() - Ak_bf)) < 1e-12


def test_btl_overflow_outside_domain():
    """BTL legs overflow when the half span passes ~88 (domain.py:1-7): the sanitized scores
    then differ from the exact ones; inside the domain they agree."""
    rng = np.random.default_rng(0)
    T, D = 64, 8
    f32 = lambda x: torch.as_tensor(x, dtype=torch.float32)
    q, k = f32(rng.normal(size=(T, D)) * 0.3), f32(rng.normal(size=(T, D)) * 0.3)
    b = f32(np.abs(rng.normal(size=(T, D))) * 0.5)
    for c, bad in ((0.5, False), (8.0, True)):
        gc = torch.cumsum(torch.full((T, D), -c, dtype=torch.float32), 0)
        cb = O.OracleCfg(bs2=32)
        _, Ab = O.btl_scores(q, k, b, gc, 0.125, cb)
        _, Al = O.btl_scores(q, k, b, gc, 0.125, cb.with_(diag="lean"))
        assert (rel(Ab, Al) > 1e-3) == bad


# ---------------------------------------------------------------- inverse
@pytest.mark.parametrize("mb", [2, 4, 8, 16, 32])
@pytest.mark.parametrize("eps", [0.0, 0.01])
def test_ladder_inverse_vs_scipy(mb, eps):
    rng = np.random.default_rng(mb)
    T = 64
    S = np.tril(rng.normal(size=(T, T)) * 0.1, -1)
    A = O.ladder_inverse(t64(S), eps, T, mb, "highest").numpy()
    M = np.eye(T) + (1 - eps) * S
    ref = scipy.linalg.solve_triangular(M, np.eye(T), lower=True, unit_diagonal=True)
    assert np.max(np.abs(A - ref)) < 1e-12
    assert np.max(np.abs(M @ A - np.eye(T))) < 1e-12
    assert np.all(np.triu(A, 1) == 0) and np.all(np.diag(A) == 1)


def test_micro_inv_brute_force():
    rng = np.random.default_rng(5)
    S = np.tril(rng.normal(size=(4, 4)), -1)
    X = O.micro_inv(t64(S)).numpy()
    # explicit inverse of a 4x4 unit lower triangular matrix by cofactors (numpy.linalg.inv)
    assert np.max(np.abs(X - np.linalg.inv(np.eye(4) + S))) < 1e-13


# ---------------------------------------------------------------- gradients
def test_autograd_vs_finite_differences_on_serial():
    """T1 (tests_gdn2/test_t1_finite_diff.py:12-33), in float64 throughout."""
    q, k, v, w, b, g, _ = rand_inputs(1, 1, 128, 16, 1)
    cfg = O.OracleCfg()
    gr = O.grad_ref(q, k, v, w, b, g, 0.25, None, cfg)
    rng = np.random.default_rng(1)
    dirs = [t64(rng.normal(size=q.shape)) for _ in range(6)]
    an = sum(float((gr[n] * d).sum()) for n, d in zip(("dq", "dk", "dv", "dw", "db", "dg"), dirs))
    sw = lambda x: x.transpose(1, 2)

    def f(s):
        qq, kk, vv, ww, bb, gg = (x + s * d for x, d in zip((q, k, v, w, b, g), dirs))
        o, hf = O.token_serial_ref(sw(qq), sw(kk), sw(vv), sw(gg), sw(bb), sw(ww), 0.25)
        return float((o * o).sum() + (hf * hf).sum())

    eps = 1e-5
    fd = (f(eps) - f(-eps)) / (2 * eps)
    assert abs(an - fd) / abs(fd) < 1e-7, (an, fd)


AB_CFGS = [
    dict(),
    dict(bs2=16),
    dict(bs2=64, mb=4),
    dict(score_bs=32, bs2=16),
    dict(diag="lean"),
    dict(wy_eps=0.05),
]


@pytest.mark.parametrize("kw", AB_CFGS)
def test_analytic_backward_matches_autograd(kw):
    """The kernel-semantics backward (bwd/mega.py + bwd/b4.py restated) equals autograd of
    the oracle forward: pins both, and the residual definitions (A, Aqk, h_pre, v_new)."""
    cfg = O.OracleCfg(**kw)
    q, k, v, w, b, g, h0 = rand_inputs(1, 2, 192, 16, 9, h0=True)
    gr = O.grad_ref(q, k, v, w, b, g, 0.25, h0, cfg)
    kf = O.kernel_forward_ref(q, k, v, w, b, g, 0.25, h0, cfg)
    ch = lambda t: O.to_chunks(t, cfg.bt)
    bw = O.backward_mega_ref(*map(ch, (q, k, v, w, b, g)), kf["A"], kf["Aqk"], kf["h_pre"], kf["v_new"],
                             ch(2 * kf["o"]), 2 * kf["h_final"], 0.25, cfg)
    for n in ("dq", "dk", "dv", "dw", "db", "dg"):
        assert rel(O.from_chunks(bw[n]), gr[n]) < 1e-9, n
    assert rel(bw["dh0"], gr["dh0"]) < 1e-9


def flat_gate_inputs(B, H, L, D, seed, tiny=0.0):
    """rand_inputs with flat gc segments in every 64-token chunk: zero gates on rows 0-4 of
    columns 0-3 (gc == 0 at the chunk start), gates equal to ``tiny`` on rows 40-63 of
    columns 4-7 (gl - gc == 0 on the tail when ``tiny`` is 0 or rounds away against gc), and
    column 8 zero over the whole chunk (gl == 0)."""
    q, k, v, w, b, g, h0 = rand_inputs(B, H, L, D, seed, gscale=0.3, h0=True)
    g = g.clone().reshape(B, H, L // 64, 64, D)
    g[..., 0:5, 0:4] = 0.0
    g[..., 40:64, 4:8] = -tiny
    g[..., :, 8] = 0.0
    return q, k, v, w, b, g.reshape(B, H, L, D), h0


def test_analytic_backward_flat_gate_segments(monkeypatch):
    """Where x = gc, gl - gc or gl is exactly 0, the derivative of exp(min(x, 0)) that
    autograd takes is 1 (torch's clamp gradient at the bound), and the analytic backward's
    masks 1{x <= 0} agree with it.  The reference backward's 1{x < 0} (bwd/mega.py:47-48)
    drops those terms; planted here, the dg check fails.  In fp32 the tail gates of 1e-9
    round away against gc and produce the same zeros: the fp32 analytic backward still
    meets the float64 autograd gradient on every chunk."""
    cfg = O.OracleCfg()
    ch = lambda t: O.to_chunks(t, 64)

    def mega(args, h0, dt):
        a = [x.to(dt) for x in args]
        kf = O.kernel_forward_ref(*a, 0.25, h0.to(dt), cfg)
        return O.backward_mega_ref(*map(ch, a), kf["A"], kf["Aqk"], kf["h_pre"], kf["v_new"],
                                   ch(2 * kf["o"]), 2 * kf["h_final"], 0.25, cfg)

    *args, h0 = flat_gate_inputs(1, 2, 128, 16, 21)
    gr = O.grad_ref(*args, 0.25, h0, cfg)
    bw = mega(args, h0, torch.float64)
    for n in ("dq", "dk", "dv", "dw", "db", "dg"):
        assert rel(O.from_chunks(bw[n]), gr[n]) < 1e-9, n
    monkeypatch.setattr(O, "exp_nonpos_grad", O.exp_nonpos)          # the strict 1{x < 0}
    assert rel(O.from_chunks(mega(args, h0, torch.float64)["dg"]), gr["dg"]) > 1e-2
    monkeypatch.undo()

    *args, h0 = flat_gate_inputs(1, 2, 256, 16, 22, tiny=1e-9)
    gr = O.grad_ref(*args, 0.25, h0, cfg)
    dg = O.from_chunks(mega(args, h0, torch.float32)["dg"]).double()
    for c in range(4):
        assert rel(dg[..., 64 * c:64 * c + 64, :], gr["dg"][..., 64 * c:64 * c + 64, :]) < 1e-5, c


@pytest.mark.parametrize("kw", [dict(), dict(bs2=16), dict(score_bs=32, bs2=16), dict(bs2=64)])
def test_b4_closed_form_vs_autograd(kw):
    cfg = O.OracleCfg(**kw)
    rng = np.random.default_rng(2)
    T, D = 64, 8
    q, k = t64(rng.normal(size=(T, D))), t64(rng.normal(size=(T, D)))
    b = t64(rng.uniform(0.2, 1, size=(T, D)))
    gc = t64(np.cumsum(-np.abs(rng.normal(size=(T, D))) * 0.1, axis=0))
    dAq, dAk = t64(rng.normal(size=(T, T))), t64(rng.normal(size=(T, T)))
    causal, strict = O.causal_masks(T)
    dAq, dAk = dAq * causal, dAk * strict
    leaves = [x.clone().requires_grad_(True) for x in (q, k, b, gc)]
    Aq, Ak = O.btl_scores(*leaves, 0.3, cfg)
    gq, gk, gb, ggc = torch.autograd.grad((Aq * dAq).sum() + (Ak * dAk).sum(), leaves)
    dq, dk, db, dgc = O.b4_exact_f64_np(q, k, b, gc, dAq, dAk, 0.3)
    for x, y in ((dq, gq), (dk, gk), (db, gb), (dgc, ggc)):
        assert np.max(np.abs(x - y.numpy())) < 1e-10
    # and the two-level B4 restatement (bwd/b4.py) agrees with the closed form
    dq2, dk2, db2, dgc2 = O._b4_2l(q, k, b, gc, dAq, dAk, 0.3, cfg, torch.matmul)
    for x, y in ((dq, dq2), (dk, dk2), (db, db2), (dgc, dgc2)):
        assert np.max(np.abs(x - y.numpy())) < 1e-10


def test_b5_reverse_cumsum():
    rng = np.random.default_rng(4)
    x = t64(rng.normal(size=(64, 8)))
    triu = torch.triu(torch.ones(64, 64))
    assert torch.allclose(triu @ x, torch.flip(torch.cumsum(torch.flip(x, [0]), 0), [0]), atol=1e-12)


def test_dot_modes():
    rng = np.random.default_rng(6)
    a, b = t64(rng.normal(size=(32, 64))), t64(rng.normal(size=(64, 16)))
    ref = a @ b
    e3 = rel(O.make_dot("bf16x3")(a, b), ref)
    e1 = rel(O.make_dot("default")(a, b), ref)
    assert e3 < 2e-5 and 1e-4 < e1 < 3e-2 and e3 < e1
    x = torch.tensor([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -3.14159])
    assert torch.equal(O.bf16_round(x), x.float().bfloat16().double())


def test_causality_of_gradient():
    """T5 causality (tests_gdn2/test_t5_grad_vs_reference.py:41-48): g beyond p does not
    change dq before p."""
    q, k, v, w, b, g, _ = rand_inputs(1, 1, 128, 16, 2)
    cfg = O.OracleCfg()
    p = 96
    g2 = g.clone()
    g2[:, :, p] -= 1.0

    def dq_o_only(gg):       # loss on o only, as in the reference test
        lv = [x.clone().requires_grad_(True) for x in (q, k, v, w, b, gg)]
        o, _ = O.forward_ref(*lv, 0.25, None, cfg)
        return torch.autograd.grad((o * o).sum(), lv[0])[0]
    assert torch.equal(dq_o_only(g)[:, :, :p], dq_o_only(g2)[:, :, :p])


# ---------------------------------------------------------------- planted mistakes
def test_planted_mistakes_are_caught(monkeypatch):
    """Each plausible slip in the oracle must fail one of the pins above."""
    q, k, v, w, b, g, h0 = rand_inputs(1, 1, 128, 16, 8, h0=True)
    sw = lambda x: x.transpose(1, 2)
    os_, hs = O.token_serial_ref(sw(q), sw(k), sw(v), sw(g), sw(b), sw(w), 0.25, h0)
    cfg = O.OracleCfg()

    def fwd_err():
        o, hf = O.forward_ref(q, k, v, w, b, g, 0.25, h0, cfg)
        return max(rel(o, sw(os_)), rel(hf, hs))

    assert fwd_err() < 1e-10
    orig_scan, orig_scores, orig_wy = O.inter_chunk_scan_ref, O.blr_scores_ref, O.recompute_wy_ref

    def scan_sign(Aqk, wp, u, kg, qg, gl, scale, h0_, cfg_, dot=None):     # v_new = u + wp h
        return orig_scan(Aqk, -wp, u, kg, qg, gl, scale, h0_, cfg_, dot)
    monkeypatch.setattr(O, "inter_chunk_scan_ref", scan_sign)
    assert fwd_err() > 1e-3
    monkeypatch.setattr(O, "inter_chunk_scan_ref", orig_scan)

    def scores_strict(q_, k_, b_, gc, scale, cfg_):                       # Aqk loses its diagonal
        Aq, Ak = orig_scores(q_, k_, b_, gc, scale, cfg_)
        return Aq * O.causal_masks(cfg_.bt)[1], Ak
    monkeypatch.setattr(O, "blr_scores_ref", scores_strict)
    assert fwd_err() > 1e-3
    monkeypatch.setattr(O, "blr_scores_ref", orig_scores)

    def wy_nodecay(q_, k_, v_, w_, b_, gc, A, cfg_, dot=None):            # drops e^gc in wp
        wp, u, kg, qg, gl = orig_wy(q_, k_, v_, w_, b_, gc, A, cfg_, dot)
        return (A @ (b_ * k_)), u, kg, qg, gl
    monkeypatch.setattr(O, "recompute_wy_ref", wy_nodecay)
    assert fwd_err() > 1e-3
    monkeypatch.setattr(O, "recompute_wy_ref", orig_wy)

    # slips in the ladder inverse are caught by the scipy pin (test_ladder_inverse_vs_scipy)
    S = torch.tril(torch.randn(64, 64, generator=torch.Generator().manual_seed(0)) * 0.3, -1)
    ref = torch.as_tensor(scipy.linalg.solve_triangular((torch.eye(64) + S).numpy(), np.eye(64), lower=True,
                                                        unit_diagonal=True))
    assert float((O.ladder_inverse(S, 0.0, 64, 8) - ref).abs().max()) < 1e-12
    orig_leaf, orig_dot = O.micro_inv, O.make_dot
    monkeypatch.setattr(O, "micro_inv", lambda Tm: orig_leaf(Tm).transpose(-1, -2))    # transposed leaf
    assert float((O.ladder_inverse(S, 0.0, 64, 8) - ref).abs().max()) > 1e-3
    monkeypatch.setattr(O, "micro_inv", orig_leaf)
    # operands of every merge product swapped: S21 X11 -> X11 S21, X22 M -> M X22
    monkeypatch.setattr(O, "make_dot", lambda mode: (lambda a, b_: orig_dot(mode)(b_, a)))
    assert float((O.ladder_inverse(S, 0.0, 64, 8) - ref).abs().max()) > 1e-3
    monkeypatch.setattr(O, "make_dot", orig_dot)

    # a dropped (1-eps) factor in dAkk is caught by the analytic-vs-autograd pin
    cfg_e = O.OracleCfg(wy_eps=0.05)
    gr = O.grad_ref(q, k, v, w, b, g, 0.25, h0, cfg_e)
    kf = O.kernel_forward_ref(q, k, v, w, b, g, 0.25, h0, cfg_e)
    ch = lambda t: O.to_chunks(t, 64)
    bw = O.backward_mega_ref(*map(ch, (q, k, v, w, b, g)), kf["A"], kf["Aqk"], kf["h_pre"], kf["v_new"],
                             ch(2 * kf["o"]), 2 * kf["h_final"], 0.25, cfg_e.with_(wy_eps=0.0))
    assert max(rel(O.from_chunks(bw[n]), gr[n]) for n in ("dq", "dk", "db", "dg")) > 1e-4


# ---------------------------------------------------------------- numerics helpers out of range
def test_numerics_helpers_outside_their_ranges():
    """precision.py:41-52 with jnp semantics: jnp.minimum and jnp.clip keep a NaN, the masks
    are False at NaN, nan_to_num maps NaN -> 0 and +-inf -> +-clip after the clip."""
    nan, inf = float("nan"), float("inf")
    c = 5e3
    x = torch.tensor([nan, inf, -inf, 2 * c, -2 * c, 0.5 * c, 0.0, -0.0], dtype=torch.float64)
    assert torch.equal(O.sanitize(x, c), torch.tensor([0.0, c, -c, c, -c, 0.5 * c, 0.0, 0.0], dtype=torch.float64))

    e, m = O.exp_nonpos(torch.tensor([nan, inf, -inf, 3.0, 0.0, -2.0], dtype=torch.float64))
    assert torch.isnan(e[0]) and e[1] == 1.0 and e[2] == 0.0 and e[3] == 1.0 and e[4] == 1.0
    assert abs(float(e[5]) - math.exp(-2.0)) < 1e-15
    assert m.tolist() == [0.0, 0.0, 1.0, 0.0, 0.0, 1.0]

    lo, hi = -20.0, 20.0
    e, m = O.exp_clipped(torch.tensor([nan, inf, -inf, 25.0, -25.0, 3.0, 20.0], dtype=torch.float64), lo, hi)
    assert torch.isnan(e[0])
    assert torch.allclose(e[1:], torch.tensor([math.exp(hi), math.exp(lo), math.exp(hi), math.exp(lo), math.exp(3.0),
                                               math.exp(hi)], dtype=torch.float64), rtol=1e-15, atol=0.0)
    assert m.tolist() == [0.0, 0.0, 0.0, 0.0, 0.0, 1.0, 1.0]


def test_nan_gate_is_zeroed_not_ignored(monkeypatch):
    """A NaN gate makes e^{min(gc,0)} NaN and the next sanitize point zero it: in the
    reference a NaN in g at token p of a chunk zeroes q's gated copy from p on (qg = san(q e^gc)),
    where a NaN-dropping min (fminf) would leave qg = q there.  The check fails on that slip."""
    cfg = O.OracleCfg()
    q, k, v, w, b, g, _ = rand_inputs(1, 1, 64, 8, 3)
    p = 40
    g = g.clone()
    g[..., p, 2] = float("nan")
    gc = torch.cumsum(g, -2)
    A = torch.eye(64, dtype=torch.float64)
    _, _, _, qg, _ = O.recompute_wy_ref(q, k, v, w, b, gc, A, cfg)
    assert torch.all(qg[..., p:, 2] == 0.0) and torch.all(qg[..., :p, 2] != 0.0)
    orig = O.exp_nonpos
    monkeypatch.setattr(O, "exp_nonpos", lambda x: (torch.exp(torch.nan_to_num(x, nan=0.0).clamp(max=0.0)),
                                                   (x < 0).to(x.dtype)))
    _, _, _, qg_bad, _ = O.recompute_wy_ref(q, k, v, w, b, gc, A, cfg)
    assert not torch.all(qg_bad[..., p:, 2] == 0.0)
    monkeypatch.setattr(O, "exp_nonpos", orig)


# ---------------------------------------------------------------- bt = 128 / 256 as parts of 64
def _group_forward(q, k, v, w, b, g, scale, h0, cfg, G):
    """The kernels' algebra for bt = 64 G (gdn2_kernels.hpp, Cfg::group), restated in float64
    from the chunk-64 pieces of the oracle: scores and WY inverse inside each 64-token part, then
    a scan whose parts j >= 1 erase from the damped state h_d(j) (h_d(0) = h(0),
    h_d(j+1) = e^gamma_j h_d(j) + (1 - eps) Kg_j^T v_new_j) while o and the state update use h."""
    eps = cfg.wy_eps
    c64 = cfg.with_(bt=64, score_bs=min(cfg.score_bs, 64))
    ch = lambda t: O.to_chunks(t, 64)
    qr, kr, vr, wr, br, gr = map(ch, (q, k, v, w, b, g))
    gc = O.chunk_gc(gr)
    Aqk, Akk = O.blr_scores_ref(qr, kr, br, gc, scale, c64)
    A = O.ladder_inverse(Akk, eps, 64, min(cfg.mb, 64))
    wp, u, kg, qg, gl = O.recompute_wy_ref(qr, kr, vr, wr, br, gc, A, c64)
    h, hd, outs = h0, None, []
    for c in range(qr.shape[-3]):
        j = c % G
        vn = u[..., c, :, :] - wp[..., c, :, :] @ (hd if j else h)
        outs.append(scale * qg[..., c, :, :] @ h + Aqk[..., c, :, :] @ vn)
        hn = kg[..., c, :, :].transpose(-1, -2) @ vn
        dec = torch.exp(gl[..., c, :])[..., :, None]
        if j < G - 1:
            hd = dec * (hd if j else h) + (1.0 - eps) * hn
        h = dec * h + hn
    return torch.cat(outs, -2), h


def _pair_forward(q, k, v, w, b, g, scale, h0, cfg128):
    return _group_forward(q, k, v, w, b, g, scale, h0, cfg128, 2)


@pytest.mark.parametrize("kw", [dict(wy_eps=0.05), dict(wy_eps=1e-3, bs2=64, mb=16), dict(wy_eps=0.2, score_bs=64)])
def test_bt256_equals_four_parts_with_damped_erase(kw):
    """The bt = 256 oracle (scores over 256 rows, ladder inverse over 256) equals the four-part
    algebra of the kernels, values and gradients, to float64 rounding; the pair algebra (bt 128)
    on the same inputs does not."""
    q, k, v, w, b, g, h0 = rand_inputs(1, 2, 512, 16, 42, gscale=0.05, h0=True)
    cfg = O.OracleCfg(bt=256, score_bs=256, bs2=32, mb=8).with_(**kw)
    xs = [x.clone().requires_grad_(True) for x in (q, k, v, w, b, g, h0)]
    o1, h1 = O.forward_ref(*xs[:6], 0.25, xs[6], cfg)
    g1 = torch.autograd.grad((o1 * o1).sum() + (h1 * h1).sum(), xs)
    o2, h2 = _group_forward(*xs[:6], 0.25, xs[6], cfg, 4)
    g2 = torch.autograd.grad((o2 * o2).sum() + (h2 * h2).sum(), xs)
    assert rel(o1, o2) < 1e-10 and rel(h1, h2) < 1e-10
    assert max(rel(a, b_) for a, b_ in zip(g1, g2)) < 1e-9
    if cfg.wy_eps > 0.01:
        o3, _ = _group_forward(*xs[:6], 0.25, xs[6], cfg.with_(bt=128, score_bs=min(cfg.score_bs, 128)), 2)
        assert rel(o1, o3) > 1e-4


@pytest.mark.parametrize("kw", [dict(wy_eps=0.05), dict(wy_eps=0.05, bs2=64), dict(wy_eps=1e-3, score_bs=64, mb=16),
                                dict(wy_eps=0.0)])
def test_bt128_equals_pairs_of_halves_with_damped_erase(kw):
    """The bt = 128 oracle (scores over 128 rows, ladder inverse over 128) equals the pair
    algebra of the kernels, values and gradients, to float64 rounding; dropping the damping
    from the second half's state (the plain chunk-64 recurrence) does not."""
    q, k, v, w, b, g, h0 = rand_inputs(1, 2, 384, 16, 41, gscale=0.05, h0=True)
    cfg = O.OracleCfg(bt=128, score_bs=128, bs2=32, mb=8).with_(**kw)
    xs = [x.clone().requires_grad_(True) for x in (q, k, v, w, b, g, h0)]
    o1, h1 = O.forward_ref(*xs[:6], 0.25, xs[6], cfg)
    g1 = torch.autograd.grad((o1 * o1).sum() + (h1 * h1).sum(), xs)
    o2, h2 = _pair_forward(*xs[:6], 0.25, xs[6], cfg)
    g2 = torch.autograd.grad((o2 * o2).sum() + (h2 * h2).sum(), xs)
    assert rel(o1, o2) < 1e-10 and rel(h1, h2) < 1e-10
    assert max(rel(a, b_) for a, b_ in zip(g1, g2)) < 1e-9
    if cfg.wy_eps > 0.01:
        o3, h3 = O.forward_ref(*xs[:6], 0.25, xs[6], cfg.with_(bt=64, score_bs=64))
        assert rel(o1, o3) > 1e-3
