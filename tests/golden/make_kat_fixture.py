"""Copy the reference's stored known-answer data for the GDN-2 recurrence into fixtures.

Source (data only, read in this container; nothing from it is executed):
``numerical/experiments/2026-10-17/controlled-rounding/inputs-seed{0,1,2}.npz`` -- float32
q,k,v,w,b,g (1,256,1,4) in (B,L,H,D), h0 (1,1,4,4), a tangent ``direction`` for v and a
``coeff`` vector (1040 = 256*4 o values + 16 h_final values) -- and ``report.json``, whose
80-digit Decimal oracle gives, per seed, the objective and its derivative along ``direction``
for two objectives over y = [o.ravel(), h_final.ravel()] at scale 0.5:
``natural`` = 0.5*sum(y^2) and ``cancellation_stress`` = sum(coeff*y).

Writes ``kat_d4_seed{s}.npz`` (arrays re-saved with numpy, no pickles) and ``kat_d4.json``.
"""
import json
import sys
from pathlib import Path

import numpy as np

SRC = Path("/root/reference/numerical/experiments/2026-10-17/controlled-rounding")
OUT = Path(__file__).resolve().parent


def main():
    if not SRC.exists():
        sys.exit(f"{SRC} not found")
    rep = json.loads((SRC / "report.json").read_text())
    cases = {}
    for seed in (0, 1, 2):
        d = np.load(SRC / f"inputs-seed{seed}.npz", allow_pickle=False)
        np.savez_compressed(OUT / f"kat_d4_seed{seed}.npz", **{k: np.asarray(d[k]) for k in d.files})
        for c in rep["cases"]:
            if c.get("seed") == seed and "mode" in c:
                cases[f"{seed}/{c['mode']}"] = dict(value=c["oracle_value_decimal"],
                                                    gradient=c["oracle_gradient_decimal"],
                                                    input_sha256=c["input_sha256"])
    meta = dict(source=str(SRC.relative_to("/root/reference")), scale=0.5, layout="BLHD",
                objectives={"natural": "0.5*sum(y^2)", "cancellation_stress": "sum(coeff*y)"},
                y="concat(o.ravel(), h_final.ravel())", derivative="d/dtheta at 0 of v + theta*direction",
                cases=cases)
    (OUT / "kat_d4.json").write_text(json.dumps(meta, indent=1))
    print(f"wrote {len(cases)} cases")


if __name__ == "__main__":
    main()
