"""bt = 128 (the reference's default and PROD chunk) against the float64 oracle run at bt = 128.

The kernels run a 128-token chunk as two 64-token halves; with wy_eps > 0 the second half
erases from the damped state e^gamma_a h + (1 - eps) Kg_a^T v_new_a (gdn2_kernels.hpp,
Cfg::group), which is the block form of the 128 chunk's WY inverse (bt = 256: four parts).  The oracle computes the
128 chunk directly (its own two-level scores, ladder inverse over 128 rows, scan), so these
tests pin that algebra (measured ~4e-7 rel-L2); as a control, the chunk-64 operator with the
same eps = 0.05 differs from the bt = 128 oracle by more than twice the gate (~5e-3).
"""
import numpy as np
import pytest
import torch

from conftest import mk_inputs, rel_l2
from test_gpu_parity import GATE, NAMES, banner, base_cfg, compare, oracle_grad, to_dev

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")


def cfg128(**kw):
    d = dict(bt=128, bc=64, score_bs=128, bs2=32, mb=8)
    d.update(kw)
    return base_cfg(**d)


def grad(cfg, scale, arrs, h0, ckpt=None, dtype=torch.float32):
    from atomic_gdn2 import make_blr_trainable
    xs = [t.requires_grad_(True) for t in to_dev(arrs, dtype)]
    h0t = torch.from_numpy(h0).cuda().requires_grad_(True)
    o, hf = make_blr_trainable(cfg, scale, state_ckpt=ckpt)(*xs, h0t)
    gr = torch.autograd.grad((o * o).sum() + (hf * hf).sum(), xs + [h0t])
    torch.cuda.synchronize()
    out = dict(o=o.detach(), h_final=hf.detach())
    out.update(zip(NAMES + ("dh0",), gr))
    return out


CASES = [
    dict(wy_eps=1e-3),                                   # the PROD geometry's damping
    dict(wy_eps=0.05, bs2=64),                           # strong damping, whole-half BTL blocks
    dict(wy_eps=0.05, score_bs=64, mb=16),
    dict(wy_eps=0.0, bs2=64),                            # the reference's published speed profile
    dict(wy_eps=0.02, score_bs=32, bs2=16, mb=4),
    dict(wy_eps=0.05, diag="lean"),
]


@pytest.mark.parametrize("kw", CASES, ids=lambda kw: ",".join(f"{k}={v}" for k, v in kw.items()))
@pytest.mark.parametrize("D", [64, 128])
def test_bt128_matches_oracle(kw, D):
    banner(f"bt=128 vs oracle {kw} D={D}")
    cfg = cfg128(**kw)
    scale = D ** -0.5
    arrs = mk_inputs(1, 384, 2, D, 31, g=0.05, layout="bhld")       # three 128-token chunks
    h0 = (np.random.default_rng(32).normal(size=(1, 2, D, D)) * 0.1).astype(np.float32)
    hip = grad(cfg, scale, arrs, h0)
    ref = oracle_grad(cfg, scale, arrs, h0)
    errs = compare(hip, ref, GATE, names=("o", "h_final") + NAMES + ("dh0",))
    banner(f"bt=128 max rel-L2 {max(errs.values()):.2e}")


def test_damping_makes_bt128_a_different_operator():
    """Control for the test above: with eps = 0.05 the chunk-64 operator is not the bt = 128
    one, beyond the parity gate, so matching the bt = 128 oracle is not automatic."""
    banner("bt=64 vs bt=128 operators under eps = 0.05")
    scale = 128 ** -0.5
    arrs = mk_inputs(1, 256, 1, 128, 33, g=0.05, layout="bhld")
    h0 = np.zeros((1, 1, 128, 128), np.float32)
    r128 = oracle_grad(cfg128(wy_eps=0.05), scale, arrs, h0)
    hip64 = grad(base_cfg(wy_eps=0.05), scale, arrs, h0)
    assert max(rel_l2(hip64[n], r128[n]) for n in ("o",) + NAMES) > 2 * GATE


def test_prod_defaults_run_and_match_oracle():
    """make_cfg() as the reference ships it (bt 128, score_bs 128, bs2 32, mb 8, wy_eps 1e-3,
    solve / backward products bf16x3) runs and matches the oracle."""
    from atomic_gdn2 import make_cfg
    banner("PROD defaults")
    cfg = make_cfg()
    assert cfg.bt == 128 and cfg.wy_eps == 1e-3
    scale = 128 ** -0.5
    arrs = mk_inputs(2, 256, 2, 128, 34, g=0.05, layout="bhld")
    h0 = (np.random.default_rng(35).normal(size=(2, 2, 128, 128)) * 0.1).astype(np.float32)
    hip = grad(cfg, scale, arrs, h0)
    compare(hip, oracle_grad(cfg, scale, arrs, h0), GATE, names=("o", "h_final") + NAMES + ("dh0",))


def test_bt128_checkpoints_segments_and_forward_only():
    """Every checkpoint interval gives the same bits (odd ones are rounded up to whole pairs);
    keeping every chunk's state is rejected with wy_eps > 0; four 128-chunks as two segments
    match the oracle; the no-grad forward equals the training forward bit for bit."""
    from atomic_gdn2 import make_blr_trainable
    banner("bt=128 checkpoints / segments / forward-only")
    cfg = cfg128(wy_eps=0.03, max_chunks_per_call=2)
    scale = 128 ** -0.5
    arrs = mk_inputs(1, 512, 2, 128, 36, g=0.05, layout="bhld")
    h0 = (np.random.default_rng(37).normal(size=(1, 2, 128, 128)) * 0.1).astype(np.float32)
    ref = grad(cfg, scale, arrs, h0, ckpt=2)
    for ck in (1, 3, 4, 8):
        got = grad(cfg, scale, arrs, h0, ckpt=ck)
        for n in ref:
            assert torch.equal(got[n], ref[n]), (ck, n)
    with pytest.raises(ValueError, match="state_ckpt"):
        grad(cfg, scale, arrs, h0, ckpt=0)
    compare(ref, oracle_grad(cfg, scale, arrs, h0), GATE, names=("o", "h_final") + NAMES + ("dh0",))
    with torch.no_grad():
        o, hf = make_blr_trainable(cfg, scale)(*to_dev(arrs), torch.from_numpy(h0).cuda())
    torch.cuda.synchronize()
    assert torch.equal(o, ref["o"]) and torch.equal(hf, ref["h_final"])


@pytest.mark.parametrize("kw", [dict(score_bs=256, bs2=32), dict(score_bs=128, bs2=64, mb=16)],
                         ids=lambda kw: ",".join(f"{k}={v}" for k, v in kw.items()))
def test_bt256_undamped_matches_oracle(kw):
    """bt = 256 with wy_eps = 0 (the undamped operator, which the kernels run as 64-token chunks)
    against the float64 oracle run at bt = 256 (its own two-level scores and 256-row ladder
    inverse)."""
    from atomic_gdn2 import make_blr_trainable
    D = 128
    cfg = base_cfg(**{**dict(bt=256, bc=128, mb=8, wy_eps=0.0), **kw})
    banner(f"bt=256 vs oracle {kw}")
    scale = D ** -0.5
    arrs = mk_inputs(1, 512, 2, D, 33, g=0.05, layout="bhld")       # two 256-token chunks
    h0 = (np.random.default_rng(4).standard_normal((1, 2, D, D)) * 0.1).astype(np.float32)
    hip = grad(cfg, scale, arrs, h0)
    compare(hip, oracle_grad(cfg, scale, arrs, h0), GATE, ("o", "h_final") + NAMES + ("dh0",))


@pytest.mark.parametrize("eps", [0.02, 1e-3])
def test_bt256_damped_gate_gradient_per_chunk(eps):
    """dg chunk by chunk at damped bt = 256: the parts 1 and 2 of a big chunk carry the extra
    decay term sum_v EZ(j+1) Delta(j) (gdn2_kernels.hpp, Cfg::group), which lands as a constant
    per column on the chunk's rows after the reverse cumsum.  The aggregate rel-L2 of dg is
    dominated by the last chunk's large gradient, so a wrong term in an earlier part (an EZ
    taken from another value block: 3.6e-3 on one chunk, 3.5e-5 in aggregate) shows only per
    chunk.  fp32 puts every chunk within ~1e-6 of the oracle; the bar is 1e-4."""
    from atomic_gdn2 import make_blr_trainable
    from oracle import gdn2_oracle as O
    banner(f"bt=256 damped dg per chunk, eps={eps}")
    D = 128
    cfg = base_cfg(bt=256, bc=128, score_bs=128, bs2=32, mb=8, wy_eps=eps)
    arrs = mk_inputs(1, 512, 2, D, 77, g=0.05, layout="bhld")          # two 256-token chunks
    xs = [t.requires_grad_(True) for t in to_dev(arrs)]
    o, hf = make_blr_trainable(cfg, D ** -0.5, state_ckpt=4)(*xs)
    dg = torch.autograd.grad((o * o).sum() + (hf * hf).sum(), xs)[5].double().cpu()
    t = [torch.from_numpy(np.asarray(a, np.float64)) for a in arrs]
    ref = O.grad_ref(*t, D ** -0.5, None, O.OracleCfg.from_cfg(cfg))["dg"]
    errs = [rel_l2(dg[:, :, 64 * c:64 * (c + 1)], ref[:, :, 64 * c:64 * (c + 1)]) for c in range(8)]
    banner(f"bt=256 damped dg per chunk: {['%.1e' % e for e in errs]}")
    assert max(errs) < 1e-4, errs


@pytest.mark.parametrize("which", ["make_cfg", "bt256"])
def test_damped_big_chunks_bf16_inputs_forward(which):
    """bf16 inputs at the damped bt = 128 of make_cfg() and at a damped bt = 256: the no-grad
    forward widens them on load, equals the fp32 path on the same values bit for bit, and is
    within the gate of the float64 oracle at that chunk size."""
    from atomic_gdn2 import make_blr_trainable, make_cfg
    from oracle import gdn2_oracle as O
    cfg = make_cfg() if which == "make_cfg" else base_cfg(bt=256, bc=128, score_bs=128, bs2=64, mb=16,
                                                          wy_eps=0.02)
    banner(f"bf16 forward, damped bt={cfg.bt} eps={cfg.wy_eps}")
    D = 128
    scale = D ** -0.5
    arrs = mk_inputs(1, 512, 2, D, 38, g=0.05, layout="bhld")
    xb = [t.to(torch.bfloat16) for t in to_dev(arrs)]
    h0 = torch.randn(1, 2, D, D, device="cuda", generator=torch.Generator("cuda").manual_seed(39)) * 0.1
    fn = make_blr_trainable(cfg, scale)
    with torch.no_grad():
        ob, hb = fn(*xb, h0)
        of, hf = fn(*[t.float() for t in xb], h0)
    torch.cuda.synchronize()
    assert ob.dtype == torch.float32 and torch.equal(ob, of) and torch.equal(hb, hf)
    t = [x.double().cpu() for x in xb]
    ro, rh = O.forward_ref(*t, scale, h0.double().cpu(), O.OracleCfg.from_cfg(cfg))
    eo, eh = rel_l2(ob, ro), rel_l2(hb, rh)
    banner(f"bf16 damped bt={cfg.bt} rel-L2 o {eo:.2e} h {eh:.2e}")
    assert eo < GATE and eh < GATE


BT256 = [
    dict(wy_eps=1e-3),                                   # the legacy bt = 256 presets' damping
    dict(wy_eps=0.05, bs2=64, mb=16),                    # strong damping
    dict(wy_eps=0.02, score_bs=64, bs2=16, mb=4),
]


@pytest.mark.parametrize("kw", BT256, ids=lambda kw: ",".join(f"{k}={v}" for k, v in kw.items()))
@pytest.mark.parametrize("D", [64, 128])
def test_bt256_damped_matches_oracle(kw, D):
    """bt = 256 with wy_eps > 0: four 64-token parts whose erase terms read the damped state
    (the forward carries it beside the true state; the backward carries the damping
    correction's cotangent across the parts and its gate-gradient term), against the float64
    oracle run at bt = 256 over 256-row chunks."""
    cfg = base_cfg(**{**dict(bt=256, bc=128, score_bs=256, bs2=32, mb=8), **kw})
    banner(f"bt=256 damped vs oracle {kw} D={D}")
    scale = D ** -0.5
    arrs = mk_inputs(1, 768, 2, D, 34, g=0.05, layout="bhld")       # three 256-token chunks
    h0 = (np.random.default_rng(35).standard_normal((1, 2, D, D)) * 0.1).astype(np.float32)
    hip = grad(cfg, scale, arrs, h0)
    errs = compare(hip, oracle_grad(cfg, scale, arrs, h0), GATE, ("o", "h_final") + NAMES + ("dh0",))
    banner(f"bt=256 max rel-L2 {max(errs.values()):.2e}")


def test_damping_makes_bt256_a_different_operator():
    """Control for the test above: with eps = 0.2 the bt = 128 operator differs from the
    bt = 256 oracle by more than twice the gate (5.4e-3 in float64), while the bt = 256 kernels
    stay within it, so matching the bt = 256 oracle is not automatic."""
    D = 64
    arrs = mk_inputs(1, 512, 2, D, 36, g=0.05, layout="bhld")
    h0 = np.zeros((1, 2, D, D), np.float32)
    cfg256 = base_cfg(bt=256, bc=128, score_bs=256, bs2=32, mb=8, wy_eps=0.2)
    ref256 = oracle_grad(cfg256, D ** -0.5, arrs, h0)
    hip256 = grad(cfg256, D ** -0.5, arrs, h0)
    hip128 = grad(cfg128(wy_eps=0.2), D ** -0.5, arrs, h0)
    assert rel_l2(hip256["o"], ref256["o"]) <= GATE
    assert rel_l2(hip128["o"], ref256["o"]) > 2 * GATE


@pytest.mark.parametrize("ckpt", [1, 3, 4, 8])
def test_bt256_checkpoint_intervals_agree_bitwise(ckpt):
    """The residual keeps the state every K 64-token chunks, K rounded up to a multiple of 4 so
    that each recompute block holds whole 256-token chunks; every K gives the same gradients
    bit for bit."""
    D = 128
    cfg = base_cfg(bt=256, bc=128, score_bs=256, bs2=32, mb=8, wy_eps=1e-3)
    arrs = mk_inputs(1, 1024, 2, D, 37, g=0.05, layout="bhld")
    h0 = (np.random.default_rng(38).standard_normal((1, 2, D, D)) * 0.1).astype(np.float32)
    a = grad(cfg, D ** -0.5, arrs, h0, ckpt=4)
    b = grad(cfg, D ** -0.5, arrs, h0, ckpt=ckpt)
    for n in a:
        assert torch.equal(a[n], b[n]), (ckpt, n)


# bs2 outside [16, 64]: a diagonal block of 8 tokens (pieces narrower than a 16 x 16 tile, formed
# elementwise) and diagonal blocks of 128 / 256 tokens (wider than the 64-token part: their end
# rows come from the anchor pre-pass)
INNER = [
    dict(bt=64, score_bs=64, bs2=8, wy_eps=0.0),
    dict(bt=64, score_bs=16, bs2=8, wy_eps=0.0),
    dict(bt=128, score_bs=128, bs2=8, wy_eps=1e-3),
    dict(bt=128, score_bs=64, bs2=8, wy_eps=0.02, diag="lean"),
    dict(bt=128, score_bs=128, bs2=128, wy_eps=1e-3),
    dict(bt=128, score_bs=128, bs2=128, wy_eps=0.0),
    dict(bt=128, score_bs=128, bs2=128, wy_eps=0.05, diag="lean"),
    dict(bt=256, score_bs=256, bs2=128, wy_eps=0.02),
    dict(bt=256, score_bs=256, bs2=256, wy_eps=0.02),
    dict(bt=256, score_bs=256, bs2=256, wy_eps=0.0, b3_dot_mode="bf16x3", solve_dot_mode="bf16x3"),
]


@pytest.mark.parametrize("kw", INNER, ids=lambda kw: ",".join(f"{k}={v}" for k, v in kw.items()))
@pytest.mark.parametrize("D", [64, 128])
def test_inner_block_sizes_match_oracle(kw, D):
    """Forward and every gradient against the float64 oracle run at the same bt / score_bs /
    bs2 over whole chunks (three chunks, h0 given)."""
    bt = kw["bt"]
    cfg = base_cfg(**{**dict(bc=bt // 2, mb=8, g_max=160.0 / kw["bs2"]), **kw})
    banner(f"inner block {kw} D={D}")
    scale = D ** -0.5
    arrs = mk_inputs(1, 3 * bt, 2, D, 41, g=0.05, layout="bhld")
    h0 = (np.random.default_rng(42).standard_normal((1, 2, D, D)) * 0.1).astype(np.float32)
    hip = grad(cfg, scale, arrs, h0)
    errs = compare(hip, oracle_grad(cfg, scale, arrs, h0), GATE, ("o", "h_final") + NAMES + ("dh0",))
    banner(f"inner block max rel-L2 {max(errs.values()):.2e}")


@pytest.mark.parametrize("bt,bs2", [(128, 128), (256, 256), (256, 128)])
def test_wide_diagonal_blocks_at_the_half_span_limit(bt, bs2):
    """|g| just under g_max = 160 / bs2 on every token: the BTL legs of a bs2-token diagonal
    block reach e^(+-0.5 |g| (bs2 - 1)) ~ e^78, within float32 only because each part measures
    its legs from the block's own first and last rows.  An anchor off by one part's gate sum
    (|g| 64 ~ 78) overflows a leg in some part (an anchor error otherwise cancels in the
    products of the legs), so this pins the anchor buffer to within the range float32 leaves."""
    D = 64
    cfg = base_cfg(bt=bt, bc=bt // 2, score_bs=bt, bs2=bs2, mb=8, wy_eps=1e-3, g_max=160.0 / bs2)
    banner(f"wide diagonal blocks at the half-span limit bt={bt} bs2={bs2}")
    scale = D ** -0.5
    q, k, v, w, b, _ = mk_inputs(1, 2 * bt, 2, D, 43, layout="bhld")
    rng = np.random.default_rng(44)
    g = (-(0.97 + 0.02 * rng.uniform(size=q.shape)) * cfg.g_max).astype(np.float32)
    assert 75.0 < float(-g.max()) * (bs2 - 1) / 2 and float(-g.min()) * (bs2 - 1) / 2 < 80.0
    arrs = (q, k, v, w, b, g)
    h0 = (rng.standard_normal((1, 2, D, D)) * 0.1).astype(np.float32)
    hip = grad(cfg, scale, arrs, h0)
    for n, x in hip.items():
        assert torch.isfinite(x).all(), n
    errs = compare(hip, oracle_grad(cfg, scale, arrs, h0), GATE, ("o", "h_final") + NAMES + ("dh0",))
    banner(f"half-span limit max rel-L2 {max(errs.values()):.2e}")
