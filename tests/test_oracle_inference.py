"""CPU pins of the oracle's inference restatements (decode_step_ref,
chunk_forward_inference_ref; reference notebooks/gdn2_v031_stage2_tpu.ipynb cell 1,
INFERENCE_V031), and the inference module's host-side validation and id conversion.

Each oracle function is checked against something it does not share code with: the token
recurrence token_serial_ref (itself pinned by the reference's stored Decimal known answers),
independently written activations, the closed form of the norm cap, separate runs per
document, and bfloat16 rounding of the float32 result.  Planted mistakes (a reset one chunk
late, the cap on the wrong axis) must fail a pin."""
import numpy as np
import pytest
import torch

from conftest import rel_l2

D_, H_ = 16, 2


def _inputs(B, H, L, D, seed):
    from atomic_gdn2.synthetic import make_inputs_np
    arrs, scale = make_inputs_np(B, H, L, D, seed=seed)
    return [torch.from_numpy(a).double() for a in arrs], scale


def _ocfg(bt=64, **kw):
    from oracle import gdn2_oracle as O
    from atomic_gdn2 import make_cfg
    d = dict(bt=bt, bc=bt // 2, score_bs=bt, bs2=32, mb=8, wy_eps=0.0, dot_mode="highest",
             solve_dot_mode="highest", b3_dot_mode="highest")
    d.update(kw)
    return O.OracleCfg.from_cfg(make_cfg(**d))


def _serial(xs, scale, h0=None):
    """token_serial_ref on head-major tensors (its own (B,L,H,D) convention and q,k,v,g,b,w order)."""
    from oracle import gdn2_oracle as O
    q, k, v, w, b, g = (x.transpose(1, 2) for x in xs)
    o, h = O.token_serial_ref(q, k, v, g, b, w, scale, h0)
    return o.transpose(1, 2), h


def _decode_all(xs, scale, h0=None, **kw):
    from oracle import gdn2_oracle as O
    B, H, L, D = xs[0].shape
    h = xs[0].new_zeros((B, H, D, D)) if h0 is None else h0
    os_ = []
    for t in range(L):
        o, h = O.decode_step_ref(*(x[:, :, t] for x in xs), h, scale, **kw)
        os_.append(o)
    return torch.stack(os_, 2), h


def test_decode_steps_equal_token_recurrence():
    xs, scale = _inputs(2, H_, 40, D_, seed=1)
    h0 = torch.randn(2, H_, D_, D_, dtype=torch.float64) * 0.1
    o, h = _decode_all(xs, scale, h0)
    os_, hs = _serial(xs, scale, h0)
    assert rel_l2(o, os_) < 1e-12 and rel_l2(h, hs) < 1e-12


def test_fused_prologue_equals_activated_inputs():
    """The notebook's R3 check (fused decode vs decode on pre-activated inputs), with the
    activations written independently in numpy float64."""
    from oracle import gdn2_oracle as O
    rng = np.random.default_rng(3)
    B, H, D = 2, 3, D_
    raw = [rng.standard_normal((B, H, D)) for _ in range(6)]
    a_log = rng.standard_normal(H) * 0.5
    dt = rng.standard_normal(D) * 0.5
    st = rng.standard_normal((B, H, D, D)) * 0.1
    nrm = lambda x: x / np.sqrt((x * x).sum(-1, keepdims=True) + 1e-6)
    sig = lambda x: 1.0 / (1.0 + np.exp(-x))
    g_act = -np.exp(a_log)[None, :, None] * np.logaddexp(raw[5] + dt[None, None, :], 0.0)
    act = [nrm(raw[0]), nrm(raw[1]), raw[2], sig(raw[3]), sig(raw[4]), g_act]
    T = lambda x: torch.from_numpy(np.asarray(x, np.float64))
    o1, h1 = O.decode_step_ref(*map(T, act), T(st), 0.7)
    o2, h2 = O.decode_step_ref(*map(T, raw), T(st), 0.7, fuse_prologue=True, a_log=T(a_log), dt_bias=T(dt))
    assert rel_l2(o1, o2) < 1e-12 and rel_l2(h1, h2) < 1e-12


def test_decode_cap_closed_form_and_nonfinite_cleanup():
    from oracle import gdn2_oracle as O
    xs, scale = _inputs(2, 3, 1, D_, seed=4)
    x1 = [x[:, :, 0] for x in xs]
    st = torch.randn(2, 3, D_, D_, dtype=torch.float64)
    _, h = O.decode_step_ref(*x1, st, scale)
    n = torch.sqrt((h * h).sum((-2, -1)))
    tau = float(n.median())
    _, hc = O.decode_step_ref(*x1, st, scale, stability_tau=tau)
    nc = torch.sqrt((hc * hc).sum((-2, -1)))
    assert torch.allclose(nc, torch.minimum(n, torch.full_like(n, tau)), rtol=1e-12)
    ratio = hc / h
    assert torch.allclose(ratio, ratio[..., :1, :1].expand_as(ratio), rtol=1e-12)   # per-head factor
    # planted mistake: one factor for the whole batch row (norm over the heads) misses the bar
    nb = torch.sqrt((h * h).sum((-3, -2, -1), keepdim=True))
    bad = h * torch.minimum(torch.ones_like(nb), tau / nb)
    assert not torch.allclose(torch.sqrt((bad * bad).sum((-2, -1))), torch.minimum(n, torch.full_like(n, tau)))
    # NaN in v of one head reaches that head's value column 5 only (through v_new[5]): the
    # column and o[5] become 0, everything else is the clean run's
    x_nan = [x.clone() for x in x1]
    x_nan[2][1, 2, 5] = float("nan")
    o0, h0_ = O.decode_step_ref(*x1, st, scale)
    o1, h1 = O.decode_step_ref(*x_nan, st, scale)
    assert o1[1, 2, 5] == 0 and torch.count_nonzero(h1[1, 2, :, 5]) == 0
    keep_h = torch.ones_like(h1, dtype=torch.bool)
    keep_h[1, 2, :, 5] = False
    keep_o = torch.ones_like(o1, dtype=torch.bool)
    keep_o[1, 2, 5] = False
    assert torch.equal(h1[keep_h], h0_[keep_h]) and torch.equal(o1[keep_o], o0[keep_o])
    # with the cap, the head's norm is NaN, the factor NaN, and the whole head's state 0
    _, h3 = O.decode_step_ref(*x_nan, st, scale, stability_tau=1e30)
    _, h3c = O.decode_step_ref(*x1, st, scale, stability_tau=1e30)
    mask = torch.ones(2, 3, dtype=torch.bool)
    mask[1, 2] = False
    assert torch.count_nonzero(h3[1, 2]) == 0 and torch.equal(h3[mask], h3c[mask])
    # +inf in v of one head reaches only its value column 5 (through v_new[5]): that column of
    # the new state and o[5] are non-finite before the cleanup, hence 0
    x_inf = [x.clone() for x in x1]
    x_inf[2][0, 1, 5] = float("inf")
    o2, h2 = O.decode_step_ref(*x_inf, st, scale)
    assert o2[0, 1, 5] == 0 and torch.count_nonzero(h2[0, 1, :, 5]) == 0


def test_decode_reset_rows_start_from_zero():
    from oracle import gdn2_oracle as O
    xs, scale = _inputs(3, 2, 1, D_, seed=5)
    x1 = [x[:, :, 0] for x in xs]
    st = torch.randn(3, 2, D_, D_, dtype=torch.float64)
    o, h = O.decode_step_ref(*x1, st, scale, reset=torch.tensor([0, 1, 0]))
    oz, hz = O.decode_step_ref(*x1, torch.zeros_like(st), scale)
    on, hn = O.decode_step_ref(*x1, st, scale)
    assert torch.equal(o[1], oz[1]) and torch.equal(h[1], hz[1])
    assert torch.equal(o[[0, 2]], on[[0, 2]]) and torch.equal(h[[0, 2]], hn[[0, 2]])


@pytest.mark.parametrize("bt,L", [(64, 192), (64, 2 * 64 + 37), (64, 29), (128, 256 + 17)])
def test_prefill_equals_token_recurrence(bt, L):
    from oracle import gdn2_oracle as O
    xs, scale = _inputs(2, H_, L, D_, seed=6)
    h0 = torch.randn(2, H_, D_, D_, dtype=torch.float64) * 0.1
    o, h = O.chunk_forward_inference_ref(*xs, scale, _ocfg(bt), h0=h0)
    os_, hs = _serial(xs, scale, h0)
    assert rel_l2(o, os_) < 1e-9 and rel_l2(h, hs) < 1e-9


def _doc_ids(B, L, starts):
    ids = torch.zeros(B, L, dtype=torch.int64)
    for b, ss in enumerate(starts):
        for s in ss:
            ids[b, s:] += 1
    return ids


@pytest.mark.parametrize("bt,L,starts", [
    (64, 256, [[64, 192], [128]]),            # chunk-aligned boundaries, different per row
    (64, 3 * 64 + 40, [[128, 64 * 3 + 11], []]),   # one in the tail (token granularity)
    (128, 384 + 20, [[256], [128, 384 + 5]]),
])
def test_prefill_resets_equal_separate_documents(bt, L, starts):
    """Each document run on its own (token recurrence from a zero state; the first from h0),
    outputs concatenated, equals the prefill with the documents' ids."""
    from oracle import gdn2_oracle as O
    B = len(starts)
    xs, scale = _inputs(B, H_, L, D_, seed=7)
    h0 = torch.randn(B, H_, D_, D_, dtype=torch.float64) * 0.1
    ids = _doc_ids(B, L, starts)
    o, h = O.chunk_forward_inference_ref(*xs, scale, _ocfg(bt), h0=h0, segment_ids=ids)
    for b in range(B):
        cuts = [0] + starts[b] + [L]
        hb = h0[b:b + 1]
        pieces = []
        for i, (a, c) in enumerate(zip(cuts[:-1], cuts[1:])):
            ob, hb = _serial([x[b:b + 1, :, a:c] for x in xs], scale, hb if i == 0 else None)
            pieces.append(ob)
        assert rel_l2(o[b:b + 1], torch.cat(pieces, 2)) < 1e-9
        assert rel_l2(h[b:b + 1], hb) < 1e-9
    # planted mistake: the state reset one chunk late fails the same comparison
    late = _doc_ids(B, L, [[s + bt for s in ss if s + bt < L] for ss in starts])
    o_bad, _ = O.chunk_forward_inference_ref(*xs, scale, _ocfg(bt), h0=h0, segment_ids=late)
    assert rel_l2(o_bad, o) > 1e-3


def test_prefill_bf16_state_is_the_rounded_fp32_state():
    from oracle import gdn2_oracle as O
    xs, scale = _inputs(1, H_, 128, D_, seed=8)
    _, h32 = O.chunk_forward_inference_ref(*xs, scale, _ocfg(64))
    _, h16 = O.chunk_forward_inference_ref(*xs, scale, _ocfg(64), state_bf16=True)
    assert torch.equal(h16, O.bf16_round(h32))


def test_prefill_cap_closed_form():
    from oracle import gdn2_oracle as O
    xs, scale = _inputs(2, H_, 128 + 3, D_, seed=9)
    _, h = O.chunk_forward_inference_ref(*xs, scale, _ocfg(64))
    n = torch.sqrt((h * h).sum((-2, -1)))
    tau = float(n.min()) * 0.5
    _, hc = O.chunk_forward_inference_ref(*xs, scale, _ocfg(64), stability_tau=tau)
    assert torch.allclose(torch.sqrt((hc * hc).sum((-2, -1))), torch.full_like(n, tau), rtol=1e-12)


# ---------------------------------------------------------------- host side of the module
def test_cu_seqlens_to_segment_ids_known_answers():
    from atomic_gdn2.inference import _segment_ids_from_cu_seqlens as f
    ids = f([0, 3, 7, 10], 2, 10, "cpu")
    assert ids.tolist() == [[0, 0, 0, 1, 1, 1, 1, 2, 2, 2]] * 2
    per_row = f(torch.tensor([[0, 5, 10], [0, 2, 10]]), 2, 10, "cpu")
    assert per_row.tolist() == [[0] * 5 + [1] * 5, [0, 0] + [1] * 8]
    assert f([0, 10], 1, 10, "cpu").tolist() == [[0] * 10]


def _cpu_inputs(B=1, H=2, L=128, D=64, g=-0.1):
    x = torch.randn(B, H, L, D) * 0.1
    return [x, x, x, x, x, torch.full((B, H, L, D), g)]


def test_prefill_validation_errors():
    from atomic_gdn2 import make_cfg
    from atomic_gdn2.inference import chunk_forward_inference as cfi
    cfg = make_cfg(bt=64, bc=32, score_bs=64, bs2=16, mb=8, g_max=160.0 / 16)
    xs = _cpu_inputs()
    seg = torch.zeros(1, 128, dtype=torch.int64)
    seg[:, 70:] = 1                                            # inside chunk 1
    with pytest.raises(ValueError, match="boundary inside chunk 1 of batch row 0"):
        cfi(*xs, 1.0, cfg, segment_ids=seg)
    with pytest.raises(ValueError, match="outside the layer domain"):
        cfi(*_cpu_inputs(g=-50.0), 1.0, cfg)
    with pytest.raises(ValueError, match="not both"):
        cfi(*xs, 1.0, cfg, segment_ids=torch.zeros(1, 128, dtype=torch.int64), cu_seqlens=[0, 64, 128])
    with pytest.raises(ValueError, match="state_dtype"):
        cfi(*xs, 1.0, cfg, state_dtype=torch.float16)
    with pytest.raises(ValueError, match="h0.shape"):                 # checked before any kernel reads it
        cfi(*xs, 1.0, cfg, h0=torch.zeros(1, 2, 64, 32))
    with pytest.raises(RuntimeError, match="ROCm device"):     # valid call: no CPU fallback
        cfi(*xs, 1.0, cfg)


def test_decode_validation_errors():
    from atomic_gdn2.inference import decode_step, LayerInputs
    x = torch.zeros(2, 3, 64)
    st = torch.zeros(2, 3, 64, 64)
    with pytest.raises(ValueError, match="pass either"):
        decode_step(x, x, x, x, x, x)
    with pytest.raises(ValueError, match="scale must be a concrete Python float"):
        decode_step(x, x, x, x, x, x, st, scale=torch.tensor(1.0))
    with pytest.raises(ValueError, match="stability_tau must be"):
        decode_step(x, x, x, x, x, x, st, stability_tau=torch.tensor(1.0))
    with pytest.raises(ValueError, match="state must be"):
        decode_step(x, x, x, x, x, x, torch.zeros(2, 3, 64, 32))
    with pytest.raises(ValueError, match="fuse_prologue=True requires"):
        decode_step(x, x, x, x, x, x, st, fuse_prologue=True)
    with pytest.raises(RuntimeError, match="ROCm device"):
        decode_step(inputs=LayerInputs(x, x, x, x, x, x), state=st)
    with pytest.raises(ValueError, match="w: expected"):
        LayerInputs(x, x, x, torch.zeros(2, 3, 32), x, x).validate(64, 64)
