"""The persistent bwd_wy's later rounds against the float64 oracle.

bwd_wy at D = 128 with the BTL diagonal runs one workgroup per CU, each walking the chunks
blockIdx.x, + gridDim.x, ...; from its second chunk on, a workgroup's dO and v_new arrive in
LDS by a DMA issued during the previous chunk's B4, its gc comes from an in-wave cumsum, and
its arguments and lane indices are re-read in every iteration (gdn2_bwd.hip).  The other small
GPU tests launch fewer chunks than the device has CUs, so they run only first rounds.  B3 H3
L2048 is 288 chunks of 64: on a 256-CU MI355X the workgroups of chunks 0..31 also take chunks
256..287, the (b, h) sequence 8.  That sequence and one from the first round are compared
with the float64 oracle run on each alone, for the geometries and dot modes that instantiate
the persistent kernel (standard and general piece lists, eps > 0, bt = 128 pairs, bf16x3).
"""
import pytest
import torch

from conftest import rel_l2
from test_gpu_parity import GATE, NAMES, banner, base_cfg, hip_grad, oracle_grad

pytestmark = pytest.mark.gpu

B, H, L, D = 3, 3, 2048, 128


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")


CASES = [
    dict(),                                                   # standard pieces, highest
    dict(bs2=16),                                             # general piece list
    dict(score_bs=32, bs2=16, mb=4),
    dict(wy_eps=0.01),
    dict(dot_mode="bf16x3", solve_dot_mode="bf16x3", b3_dot_mode="bf16x3"),
    dict(bt=128, bc=64, score_bs=128, bs2=32, wy_eps=1e-3),   # pairs of 64-token halves
]


@pytest.mark.parametrize("kw", CASES, ids=lambda kw: ",".join(f"{k}={v}" for k, v in kw.items()) or "base")
def test_persistent_later_rounds_match_oracle(kw):
    from atomic_gdn2.synthetic import make_inputs_np
    ncu = torch.cuda.get_device_properties(0).multi_processor_count
    nchunks = B * H * (L // 64)
    if ncu >= nchunks:
        pytest.skip(f"{ncu} CUs: {nchunks} chunks fit in one round")
    late = ncu // (L // 64)                       # first sequence whose chunks a workgroup takes second
    seqs = [(late // H, late % H), (0, 1)]
    banner(f"persistent rounds {kw}: {nchunks} chunks on {ncu} CUs, sequences {seqs}")
    arrs, scale = make_inputs_np(B, H, L, D, seed=5)
    cfg = base_cfg(**kw)
    hip = hip_grad(cfg, scale, arrs)
    for n, t in hip.items():
        assert torch.isfinite(t).all(), n
    for bi, hi in seqs:
        ref = oracle_grad(cfg, scale, [a[bi:bi + 1, hi:hi + 1] for a in arrs])
        errs = {n: rel_l2(hip[n][bi:bi + 1, hi:hi + 1], ref[n]) for n in ("o", "h_final") + NAMES}
        banner(f"  sequence {(bi, hi)} max rel-L2 {max(errs.values()):.2e}")
        assert max(errs.values()) <= GATE, (bi, hi, errs)
