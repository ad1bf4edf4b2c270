"""Write the config-1 golden fixture with the float64 CPU oracle.

Config 1: (B,H,L,D) = (1,2,256,128), chunk 64, wy_eps = 0, zero h0, synthetic seed 0
(atomic_gdn2.synthetic), loss sum(o^2) + sum(h_final^2).  Stored (float32): o, h_final and
the six input gradients, plus chunk-0/head-0 intermediates Akk, A, Wp, U in kernel semantics,
and the SHA-256 of the generated inputs so that the generator itself is pinned.

Run from the repository root: ``python tests/golden/make_golden.py``.
"""
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path[:0] = [str(ROOT), str(ROOT / "atomic-ops_amd")]

from oracle import gdn2_oracle as O  # noqa: E402
from atomic_gdn2.synthetic import make_inputs_np, inputs_sha256  # noqa: E402

OUT = Path(__file__).resolve().parent / "config1_seed0.npz"


def main():
    arrs, scale = make_inputs_np(1, 2, 256, 128, seed=0)
    t = [torch.from_numpy(a).double() for a in arrs]
    cfg = O.OracleCfg(bt=64, score_bs=64, bs2=32, mb=8, wy_eps=0.0)
    gr = O.grad_ref(*t, scale, None, cfg)
    st = O.wy_stage_ref(*t, scale, cfg)
    f = lambda x: x.detach().numpy().astype(np.float32)
    np.savez_compressed(
        OUT, sha256=np.array(inputs_sha256(arrs)), scale=np.array(scale),
        o=f(gr["o"]), h_final=f(gr["h_final"]),
        **{n: f(gr[n]) for n in ("dq", "dk", "dv", "dw", "db", "dg")},
        akk00=f(st["Akk"][0, 0, 0]), A00=f(st["A"][0, 0, 0]), wp00=f(st["wp"][0, 0, 0]),
        u00=f(st["u"][0, 0, 0]))
    print(OUT, OUT.stat().st_size)


if __name__ == "__main__":
    main()
