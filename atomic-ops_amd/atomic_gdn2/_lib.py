"""ctypes binding of ``libgdn2_hip.so`` (declared in ``include/gdn2.h``).

The library is built in-tree by ``atomic-ops_amd/build_lib.py``.  There is no fallback:
if the library is missing or fails to load, every operator call raises.
``torch`` is imported first so that the library binds to the HIP runtime torch already
loaded (both carry the SONAME ``libamdhip64.so.7``): one runtime, one set of streams.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (must be loaded before the HIP library)

LIB_PATH = Path(os.environ.get("GDN2_LIB", Path(__file__).resolve().parent / "_lib" / "libgdn2_hip.so"))

DOT_IDS = {"highest": 0, "bf16x3": 1, "default": 2}
DIAG_IDS = {"btl": 0, "lean": 1}
RES_NAMES = ("aqk", "A", "h_pre", "v_new", "wp", "kg", "qg", "gl")
# per residual: (rows, cols) of the stored matrix per chunk (T = bt, D = head dim), whether it
# is stored in fragment layout, and whether it is the transpose of the named quantity
RES_STORAGE = {"aqk": ("T", "T", True, False), "A": ("T", "T", False, False),
               "h_pre": ("D", "D", True, True), "v_new": ("D", "T", True, True),
               "wp": ("T", "D", True, False), "kg": ("T", "D", True, False),
               "qg": ("T", "D", True, False), "gl": (None, "D", False, False)}
KERNEL_NAMES = ("wy_fwd", "scan_fwd", "scan_bwd", "bwd_state", "bwd_wy", "out_fwd", "bwd_pre", "bwd_state_rc",
                "decode", "anchors")
ABI_VERSION = 3
STATUS = {0: "ok", 1: "invalid argument", 2: "unsupported configuration", 3: "HIP error"}

_c_int, _c_dbl, _c_size, _vp = ctypes.c_int32, ctypes.c_double, ctypes.c_size_t, ctypes.c_void_p


class Gdn2Desc(ctypes.Structure):
    """``struct gdn2_desc`` (include/gdn2.h)."""
    _fields_ = [("B", _c_int), ("H", _c_int), ("L", _c_int), ("D", _c_int),
                ("bt", _c_int), ("score_bs", _c_int), ("bs2", _c_int), ("mb", _c_int),
                ("diag", _c_int), ("dot_mode", _c_int), ("solve_dot_mode", _c_int),
                ("b3_dot_mode", _c_int), ("seq_ld", _c_int), ("state_ckpt", _c_int),
                ("scale", _c_dbl), ("wy_eps", _c_dbl), ("clip", _c_dbl), ("diff_clip", _c_dbl)]


class Gdn2DecodeDesc(ctypes.Structure):
    """``struct gdn2_decode_desc`` (include/gdn2.h)."""
    _fields_ = [("B", _c_int), ("H", _c_int), ("D", _c_int), ("n_tok", _c_int), ("seq_ld", _c_int),
                ("in_dtype", _c_int), ("out_dtype", _c_int), ("state_dtype", _c_int),
                ("fuse_prologue", _c_int), ("cap", _c_int), ("scale", _c_dbl), ("stability_tau", _c_dbl)]


class Gdn2Error(RuntimeError):
    pass


_LIB = None


def lib():
    """Load the HIP library once; raise loudly if it is not there."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise Gdn2Error(f"{LIB_PATH} is not built; run `python atomic-ops_amd/build_lib.py`")
        L = ctypes.CDLL(str(LIB_PATH))
        P = ctypes.POINTER
        L.gdn2_abi_version.restype = _c_int
        L.gdn2_last_error.restype = ctypes.c_char_p
        L.gdn2_residual_layout.argtypes = [P(Gdn2Desc), P(_c_size), P(_c_size)]
        L.gdn2_fwd_workspace_bytes.argtypes = [P(Gdn2Desc), _c_int]
        L.gdn2_fwd_workspace_bytes.restype = _c_size
        L.gdn2_bwd_workspace_bytes.argtypes = [P(Gdn2Desc)]
        L.gdn2_bwd_workspace_bytes.restype = _c_size
        L.gdn2_fwd.argtypes = [P(Gdn2Desc)] + [_vp] * 12
        L.gdn2_fwd_bf16.argtypes = [P(Gdn2Desc)] + [_vp] * 12
        L.gdn2_fwd_noalloc.argtypes = [P(Gdn2Desc)] + [_vp] * 10
        L.gdn2_fwd_reset.argtypes = [P(Gdn2Desc), _c_int] + [_vp] * 12
        L.gdn2_decode.argtypes = [P(Gdn2DecodeDesc)] + [_vp] * 13
        L.gdn2_bwd.argtypes = [P(Gdn2Desc)] + [_vp] * 18
        L.gdn2_wy_stage.argtypes = [P(Gdn2Desc)] + [_vp] * 15
        L.gdn2_scores.argtypes = [P(Gdn2Desc)] + [_vp] * 7
        L.gdn2_debug_gemm.argtypes = [_c_int, _vp, _vp, _vp, _c_int, _c_int, _c_int, _vp]
        L.gdn2_debug_stream.argtypes = [_c_int, _vp, _vp, _c_size, _vp]
        L.gdn2_debug_mfma.argtypes = [_c_int, _c_int, _vp, _vp]
        L.gdn2_prof_begin.argtypes = [_c_int]
        L.gdn2_prof_end.argtypes = [P(_c_dbl), P(_c_int)]
        for fn in ("gdn2_residual_layout", "gdn2_fwd", "gdn2_fwd_bf16", "gdn2_fwd_noalloc", "gdn2_fwd_reset",
                   "gdn2_decode", "gdn2_bwd", "gdn2_wy_stage", "gdn2_scores", "gdn2_debug_gemm", "gdn2_debug_stream",
                   "gdn2_debug_mfma", "gdn2_prof_begin", "gdn2_prof_end"):
            getattr(L, fn).restype = _c_int
        if L.gdn2_abi_version() != ABI_VERSION:
            raise Gdn2Error("libgdn2_hip.so ABI version mismatch")
        _LIB = L
    return _LIB


def check(status: int, what: str):
    if status != 0:
        msg = lib().gdn2_last_error().decode(errors="replace")
        err = ValueError if status in (1, 2) else Gdn2Error
        raise err(f"{what}: {STATUS.get(status, status)}: {msg}")


def make_desc(cfg, B, H, L, D, scale, seq_ld=0, state_ckpt=0) -> Gdn2Desc:
    """Descriptor of one segment of L tokens; seq_ld = the full sequence length of the raw
    tensors the segment lies in (0 = L)."""
    return Gdn2Desc(B, H, L, D, cfg.bt, cfg.score_bs, cfg.bs2, cfg.mb,
                    DIAG_IDS[cfg.diag], DOT_IDS[cfg.dot_mode], DOT_IDS[cfg.solve_dot_mode],
                    DOT_IDS[cfg.b3_dot_mode], int(seq_ld), int(state_ckpt), float(scale),
                    float(cfg.wy_eps), float(cfg.clip), float(cfg.diff_clip))


def residual_layout(desc: Gdn2Desc):
    offs = (_c_size * len(RES_NAMES))()
    tot = _c_size()
    check(lib().gdn2_residual_layout(ctypes.byref(desc), offs, ctypes.byref(tot)), "gdn2_residual_layout")
    return list(offs), tot.value


def decode_residual(name, flat, B, H, nc, T, D):
    """Row-major (B, H, nc, rows, cols) tensor of one residual sub-buffer (``flat`` float32),
    un-transposed: h_pre / v_new in their natural layout."""
    from .layout import from_frag
    R, C, frag, transposed = RES_STORAGE[name]
    dim = {"T": T, "D": D}
    if R is None:
        return flat[:B * H * nc * dim[C]].reshape(B, H, nc, dim[C])
    R, C = dim[R], dim[C]
    t = flat[:B * H * nc * R * C].reshape(B, H, nc, R * C)
    t = from_frag(t, R, C) if frag else t.reshape(B, H, nc, R, C)
    return t.transpose(-1, -2) if transposed else t


def ptr(t, offset=0):
    """Device address of t (plus ``offset`` elements), or None."""
    return None if t is None else ctypes.c_void_p(t.data_ptr() + offset * t.element_size())


def stream_handle(device=None):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def prof_begin(max_launches: int):
    check(lib().gdn2_prof_begin(int(max_launches)), "gdn2_prof_begin")


def prof_end():
    ms = (_c_dbl * len(KERNEL_NAMES))()
    cnt = (_c_int * len(KERNEL_NAMES))()
    check(lib().gdn2_prof_end(ms, cnt), "gdn2_prof_end")
    return {n: (ms[i], cnt[i]) for i, n in enumerate(KERNEL_NAMES)}
