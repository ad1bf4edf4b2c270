"""The allocation-free forward (gdn2_fwd_noalloc) against gdn2_fwd with a caller workspace,
through the C ABI: bit-equal outputs on two calls in a row, the second smaller than the first
(the device scratch keeps the first call's contents), and a clear error above the scratch size."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")


def _cfg(**kw):
    from atomic_gdn2 import make_cfg
    base = dict(bt=64, bc=32, score_bs=64, bs2=32, mb=8, wy_eps=0.0, dot_mode="highest",
                solve_dot_mode="highest", b3_dot_mode="highest")
    return make_cfg(**{**base, **kw})


def _run_both(B, H, L, D, seed, with_h0, cfg=None):
    from atomic_gdn2 import _lib
    from atomic_gdn2.synthetic import make_inputs
    cfg = _cfg() if cfg is None else cfg
    print(f"[gpu-test] noalloc vs gdn2_fwd B{B} H{H} L{L} D{D} seed {seed} h0={with_h0} bt={cfg.bt} "
          f"wy_eps={cfg.wy_eps}", flush=True)
    xs, scale = make_inputs(B, H, L, D, seed=seed)
    h0 = None
    if with_h0:
        h0 = torch.randn(B, H, D, D, device="cuda", generator=torch.Generator("cuda").manual_seed(seed)) * 0.1
    desc = _lib.make_desc(cfg, B, H, L, D, scale)
    lib = _lib.lib()
    stream = _lib.stream_handle()
    o1 = torch.empty(B, H, L, D, device="cuda")
    h1 = torch.empty(B, H, D, D, device="cuda")
    ws = torch.empty(lib.gdn2_fwd_workspace_bytes(ctypes.byref(desc), 0), dtype=torch.uint8, device="cuda")
    _lib.check(lib.gdn2_fwd(ctypes.byref(desc), *map(_lib.ptr, xs), _lib.ptr(h0), _lib.ptr(o1), _lib.ptr(h1),
                            None, _lib.ptr(ws), stream), "gdn2_fwd")
    o2 = torch.full_like(o1, float("nan"))
    h2 = torch.full_like(h1, float("nan"))
    o3, h3 = torch.full_like(o1, float("nan")), torch.full_like(h1, float("nan"))
    _lib.check(lib.gdn2_fwd_noalloc(ctypes.byref(desc), *map(_lib.ptr, xs), _lib.ptr(h0), _lib.ptr(o3),
                                    _lib.ptr(h3), stream), "gdn2_fwd_noalloc")
    torch.cuda.synchronize()
    # the entry point allocates no device memory: after a warm-up call (the first call in a process
    # loads the code object that holds the scratch array, which stays resident), free device memory
    # (hipMemGetInfo) is the same before and after a call
    free0 = torch.cuda.mem_get_info()[0]
    _lib.check(lib.gdn2_fwd_noalloc(ctypes.byref(desc), *map(_lib.ptr, xs), _lib.ptr(h0), _lib.ptr(o2),
                                    _lib.ptr(h2), stream), "gdn2_fwd_noalloc")
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0
    assert torch.equal(o2, o3) and torch.equal(h2, h3)
    return (o1, h1), (o2, h2)


def test_noalloc_forward_equals_gdn2_fwd_twice_second_smaller():
    (o1, h1), (o2, h2) = _run_both(2, 3, 512, 128, 11, True)
    assert torch.isfinite(o1).all() and torch.equal(o1, o2) and torch.equal(h1, h2)
    (o1, h1), (o2, h2) = _run_both(1, 2, 192, 64, 12, False)
    assert torch.isfinite(o1).all() and torch.equal(o1, o2) and torch.equal(h1, h2)


def test_noalloc_damped_big_chunks_equal_gdn2_fwd_twice_second_smaller():
    """The reference's default geometry (make_cfg(): bt 128, wy_eps 1e-3, two damped parts per
    chunk) and a damped bt = 256 (four parts), the second call smaller than the first."""
    from atomic_gdn2 import make_cfg
    (o1, h1), (o2, h2) = _run_both(2, 2, 1024, 128, 21, True, cfg=make_cfg())
    assert torch.isfinite(o1).all() and torch.equal(o1, o2) and torch.equal(h1, h2)
    cfg256 = _cfg(bt=256, bc=128, score_bs=128, bs2=64, mb=16, wy_eps=0.02)
    (o1, h1), (o2, h2) = _run_both(1, 2, 512, 64, 22, False, cfg=cfg256)
    assert torch.isfinite(o1).all() and torch.equal(o1, o2) and torch.equal(h1, h2)


def test_noalloc_rejects_calls_above_the_scratch():
    """Buffers of the call's full size (B4 H6 L4096 D128, ~350 MB), so that nothing but the
    library's own size check stands between the call and the device: it returns
    GDN2_ERR_UNSUPPORTED naming the scratch, enqueues nothing, and leaves the outputs untouched."""
    from atomic_gdn2 import _lib
    from atomic_gdn2.synthetic import make_inputs
    B, H, L, D = 4, 6, 4096, 128
    xs, scale = make_inputs(B, H, L, D, seed=0)
    o = torch.full((B, H, L, D), 7.0, device="cuda")
    h = torch.full((B, H, D, D), 7.0, device="cuda")
    desc = _lib.make_desc(_cfg(), B, H, L, D, scale)      # 1536 chunks: ~217 MiB of workspace
    st = _lib.lib().gdn2_fwd_noalloc(ctypes.byref(desc), *map(_lib.ptr, xs), None, _lib.ptr(o), _lib.ptr(h),
                                     _lib.stream_handle())
    torch.cuda.synchronize()
    assert st == 2 and b"scratch" in _lib.lib().gdn2_last_error()
    assert bool((o == 7.0).all()) and bool((h == 7.0).all())
