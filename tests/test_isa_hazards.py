"""CPU check that the compiled gfx950 kernels keep the MFMA issue discipline: no instruction
touches an in-flight MFMA's registers (tests/mfma_hazards.py)."""
import shutil
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "tests"))


def test_scanner_flags_a_planted_hazard():
    import mfma_hazards as M
    asm = """_Zk:
\tv_mfma_f32_16x16x4_f32 v[6:9], v28, v68, v[6:9]
\ts_nop 0
\tv_mov_b32_e32 v19, v6
"""
    assert M.scan(asm)["_Zk"][0][2] == "RAW"
    ok = """_Zk:
\tv_mfma_f32_16x16x4_f32 v[6:9], v28, v68, v[6:9]
\tv_mfma_f32_16x16x4_f32 v[6:9], v29, v69, v[6:9]
\ts_nop 7
\ts_nop 7
\ts_nop 7
\tv_mov_b32_e32 v19, v6
"""
    assert M.scan(ok) == {}


@pytest.mark.skipif(shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists(),
                    reason="hipcc not available")
def test_kernels_have_no_mfma_hazards():
    import mfma_hazards as M
    found = M.check_all(verbose=False)
    assert not found, {k: v[:4] for k, v in found.items()}
