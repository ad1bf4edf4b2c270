"""Benchmark of the GDN-2 operator's gradient evaluation on one MI355X.

Workload (benchmark config 2): (B,H,L,D) = (4,6,2048,128) fp32, chunk 64, wy_eps = 0,
zero h0, synthetic seeded inputs (atomic_gdn2.synthetic); one step = forward + backward of
sum(o^2) + sum(h_final^2) w.r.t. q, k, v, w, b, g, all dot modes 'highest' (fp32 MFMA).
The timed loop runs K steps bracketed by device synchronisation, without profiling events.

Prints ONE JSON line.  ``value`` is the canonical-FLOP throughput of the whole step in
TFLOP/s (F_grad = B*H*L*(32*T*D + 18*D^2 + 4*T^2)); ``ms_per_step`` is the latency.
``roofline`` describes the dominant kernel, timed live with HIP events recorded on the launch
stream by the library (gdn2_prof_begin / gdn2_prof_end) in a second pass of K steps.
``cpu_baseline`` times the torch float32 CPU restatement of the reference algorithm
(oracle/gdn2_oracle.py) on the host cores: config 1 in full and a quarter of config 2.
Beside the headline line's fields: ``config3_sweep`` (grad-eval latency at B4 D128 for
H in {2,4,6} x L in {2048,4096}, next to the reference's published TPU v5e latencies) and
``config4_long_context_fwd`` (forward-only B8 H16 L32768 D128 with bf16 inputs, 8 calls of
4096 tokens carrying the state; tokens/s and canonical GB/s), and ``config5_e2e_lm`` (one
training step of the reference's 8-block benchmark LM around the operator, B8 L2048), and
``inference`` (decode_step and the document-reset prefill at config 4's shape).
``--no-sweep`` skips configs 3 and 4 and the inference entry points, ``--no-e2e`` config 5.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path[:0] = [str(ROOT), str(ROOT / "atomic-ops_amd")]

PEAK_FP32_MFMA = 157.3      # TFLOP/s, MI355X dense fp32 matrix
PEAK_HBM = 8000.0           # GB/s
B_, H_, L_, D_, T_ = 4, 6, 2048, 128, 64

# Algorithmic FLOPs per (batch, head, token) of the work each kernel does, in the dense
# convention of the canonical count (every T x T operand dense).  Their sum is the canonical
# F_grad minus the W recompute (2*T*D) that this implementation keeps as a residual instead.
# With state checkpoints (state_ckpt >= 1) the training forward scan also computes o (the
# output kernel does not run), and bwd_state_rc does bwd_state's reductions; the 2 D^2 per
# token of its state recompute ((K-1)/K of the chunks) is extra work, not counted.
def kernel_flops_per_token(T=T_, D=D_, fused_out=False):
    return {
        "wy_fwd": 8 * T * D,                      # Aqk, Akk, Wp, U
        "scan_fwd": 4 * D * D + (2 * T * D + 2 * D * D if fused_out else 0),   # Wp h, Kg^T v_new (+ o)
        "out_fwd": 2 * T * D + 2 * D * D,         # Aqk v_new, Qg h_pre
        "bwd_pre": 2 * T * D + 2 * D * D,         # Aqk^T dO, Qg^T dO
        "scan_bwd": 4 * D * D,                    # Kg dh, Wp^T dv_new
        "bwd_state": 6 * D * D,                   # dQg, dWp, dKg
        "bwd_state_rc": 6 * D * D,                # dQg, dWp, dKg (+ uncounted state recompute)
        "bwd_wy": 18 * T * D + 4 * T * T,         # dAqk, dA, dkb, dwv, B4; dA A^T, A^T tmp
    }


def canonical_flops(B, H, L, D, T=T_):
    n = B * H * L
    return n * (10 * T * D + 6 * D * D), n * (22 * T * D + 12 * D * D + 4 * T * T)


def canonical_bytes(B, H, L, D):
    N = B * H * L * D
    S = B * H * D * D * 4
    return 20 * N * 4 + 4 * S


def _host_cpu():
    """The host's CPU as lscpu reports it (model, sockets, cores per socket, threads per core,
    logical CPUs), plus os.cpu_count()."""
    import subprocess
    info = {"os_cpu_count": os.cpu_count()}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
    except (OSError, subprocess.SubprocessError):
        out = ""
    keys = {"Model name": "model", "Socket(s)": "sockets", "Core(s) per socket": "cores_per_socket",
            "Thread(s) per core": "threads_per_core", "CPU(s)": "logical_cpus"}
    for ln in out.splitlines():
        k, _, v = ln.partition(":")
        if k.strip() in keys:
            info[keys[k.strip()]] = v.strip()
    return info


def _median_ms_cpu(fn, reps=4, rounds=3, warm=2):
    """The reference's protocol on the host: warmups, then the median over rounds of the mean
    of reps calls."""
    for _ in range(warm):
        fn()
    per = []
    for _ in range(rounds):
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        per.append((time.perf_counter() - t0) * 1e3 / reps)
    return sorted(per)[len(per) // 2]


def cpu_baseline():
    """The oracle's chunked-WY restatement of the reference algorithm in torch float32 on the
    host CPU (forward + autograd backward of the same loss), on all os.cpu_count() threads,
    under the reference's median protocol: config 1 in full, and a quarter of config 2
    (B1 H6 L2048 D128) as the bounded sample the throughput is quoted on."""
    import torch
    from oracle import gdn2_oracle as O
    from atomic_gdn2.synthetic import make_inputs_np
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    cfg = O.OracleCfg(bt=64, score_bs=64, bs2=32, mb=8, wy_eps=0.0)

    def grad_ms(B, H, L, D):
        arrs, scale = make_inputs_np(B, H, L, D, seed=0)
        xs = [torch.from_numpy(a) for a in arrs]
        return _median_ms_cpu(lambda: O.grad_ref(*xs, scale, None, cfg))

    c1 = grad_ms(1, 2, 256, 128)
    c2 = grad_ms(1, 6, 2048, 128)
    f1 = sum(canonical_flops(1, 2, 256, 128))
    f2 = sum(canonical_flops(1, 6, 2048, 128))
    return {"value": f2 / (c2 * 1e-3) / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": "B1 H6 L2048 D128 fp32 grad-eval (1/4 of config 2), torch float32 on the host, "
                      f"median protocol (2 warmups, median of 3 rounds of 4): {c2:.1f} ms",
            "ms_per_sample": round(c2, 3), "ms_scaled_to_workload": round(c2 * 4, 3),
            "config1_full": {"shape": [1, 2, 256, 128], "ms": round(c1, 3),
                             "tflops": round(f1 / (c1 * 1e-3) / 1e12, 5)},
            "host": _host_cpu()}


# Published grad-eval latencies of the reference on TPU v5e at B4 D128 (README.md:23-30 of the
# reference, column NEW; it runs bt=128 there), by (H, L).
REF_TPU_MS = {(2, 2048): 1.701, (2, 4096): 2.943, (4, 2048): 2.702, (4, 4096): 10.493, (6, 2048): 2.888,
              (6, 4096): 13.818}


def _median_ms(fn, reps=4, rounds=3, warm=2):
    """The reference's protocol: warmups, then the median over rounds of the mean of reps calls."""
    import torch
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    per = []
    for _ in range(rounds):
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        torch.cuda.synchronize()
        per.append((time.perf_counter() - t0) * 1e3 / reps)
    return sorted(per)[len(per) // 2]


def seeds_config2(cfg):
    """Config 2 under the reference's protocol over seeds 0, 1, 2: per seed the median over 3
    rounds of 4 gradient evaluations (2 warmups), then mean and SD across the seeds."""
    import torch
    from atomic_gdn2 import make_blr_trainable
    from atomic_gdn2.synthetic import make_inputs
    per = []
    for seed in (0, 1, 2):
        (q, k, v, w, b, g), scale = make_inputs(B_, H_, L_, D_, seed=seed)
        xs = [t.requires_grad_(True) for t in (q, k, v, w, b, g)]
        fn = make_blr_trainable(cfg, scale)

        def step():
            o, hf = fn(*xs)
            return torch.autograd.grad((o, hf), xs, grad_outputs=(2.0 * o, 2.0 * hf))

        per.append(_median_ms(step))
        del xs, q, k, v, w, b, g
    mean = sum(per) / len(per)
    sd = (sum((x - mean) ** 2 for x in per) / (len(per) - 1)) ** 0.5
    return {"seeds": [0, 1, 2], "ms": [round(x, 4) for x in per], "mean_ms": round(mean, 4), "sd_ms": round(sd, 4),
            "protocol": "2 warmups, then the median over 3 rounds of the mean of 4 calls, per seed"}


def sweep_config3(cfg, seed):
    """Config 3: grad-eval latency at B4 D128, H in {2,4,6} x L in {2048,4096}
    (L=4096 runs as two segments of 32 chunks, as in the reference)."""
    import torch
    from atomic_gdn2 import make_blr_trainable
    from atomic_gdn2.synthetic import make_inputs
    out = []
    for H in (2, 4, 6):
        for L in (2048, 4096):
            (q, k, v, w, b, g), scale = make_inputs(4, H, L, 128, seed=seed)
            xs = [t.requires_grad_(True) for t in (q, k, v, w, b, g)]
            fn = make_blr_trainable(cfg, scale)

            def step():
                o, hf = fn(*xs)
                return torch.autograd.grad((o, hf), xs, grad_outputs=(2.0 * o, 2.0 * hf))

            ms = _median_ms(step)
            ff, fb = canonical_flops(4, H, L, 128)
            ref = REF_TPU_MS[(H, L)]
            out.append({"B": 4, "H": H, "L": L, "ms": round(ms, 4), "tflops": round((ff + fb) / (ms * 1e-3) / 1e12, 2),
                        "ref_tpu_v5e_ms": ref, "speedup_vs_ref": round(ref / ms, 2)})
            del xs, q, k, v, w, b, g
    return out


def state_ckpt_table(cfg, seed, ks=(0, 1, 2, 3, 4, 8, 32)):
    """Stored vs recomputed states: per state_ckpt K (0 = every chunk's state kept) the
    grad-eval latency under the median protocol, the residual size and the per-kernel HIP-event
    durations, at config 2 and at B4 H6 L4096."""
    import ctypes
    import torch
    from atomic_gdn2 import make_blr_trainable, _lib
    from atomic_gdn2.synthetic import make_inputs
    rows = []
    for (B, H, L) in ((4, 6, 2048), (4, 6, 4096)):
        (q, k, v, w, b, g), scale = make_inputs(B, H, L, 128, seed=seed)
        xs = [t.requires_grad_(True) for t in (q, k, v, w, b, g)]

        def make_step(K):
            fn = make_blr_trainable(cfg, scale, state_ckpt=K)

            def step():
                o, hf = fn(*xs)
                return torch.autograd.grad((o, hf), xs, grad_outputs=(2.0 * o, 2.0 * hf))
            return step

        steps = {K: make_step(K) for K in ks}
        # every K warmed up first, then 5 rounds that each time every K in turn (the mean of 4
        # calls), so clock and cache state are shared fairly; the median round per K
        for K in ks:
            for _ in range(3):
                steps[K]()
        torch.cuda.synchronize()
        per = {K: [] for K in ks}
        for _ in range(5):
            for K in ks:
                t0 = time.perf_counter()
                for _ in range(4):
                    steps[K]()
                torch.cuda.synchronize()
                per[K].append((time.perf_counter() - t0) * 1e3 / 4)
        for K in ks:
            step = steps[K]
            ms = sorted(per[K])[len(per[K]) // 2]
            _lib.prof_begin(4 * 16)
            for _ in range(4):
                step()
            torch.cuda.synchronize()
            prof = _lib.prof_end()
            seg = min(L, cfg.max_chunks_per_call * cfg.bt)
            desc = _lib.make_desc(cfg, B, H, seg, 128, scale, seq_ld=L, state_ckpt=K)
            offs, tot = _lib.residual_layout(desc)
            nseg = L // seg
            rows.append({"B": B, "H": H, "L": L, "state_ckpt": K, "ms": round(ms, 4),
                         "residual_mb": round(tot * nseg / 1e6, 1),
                         "state_mb": round((offs[3] - offs[2]) * nseg / 1e6, 1),
                         "kernel_us": {n: round(t / c * 1e3, 1) for n, (t, c) in prof.items() if c}})
        del xs, q, k, v, w, b, g
    return rows


def dot_mode_table(seed):
    """Config 2's gradient evaluation under each dot mode (the three set alike), the PROD
    precision mix (scores and scan fp32, solve and backward products bf16x3) at bt 64, and
    make_cfg() as the reference ships it (bt 128, wy_eps 1e-3, that mix); median protocol."""
    import torch
    from atomic_gdn2 import make_cfg, make_blr_trainable, _lib
    from atomic_gdn2.synthetic import make_inputs
    (q, k, v, w, b, g), scale = make_inputs(B_, H_, L_, D_, seed=seed)
    xs = [t.requires_grad_(True) for t in (q, k, v, w, b, g)]
    base = dict(bt=64, bc=32, score_bs=64, bs2=32, mb=8, wy_eps=0.0)
    rows = {}
    for name, cfg in (("highest", make_cfg(**base, dot_mode="highest", solve_dot_mode="highest", b3_dot_mode="highest")),
                      ("bf16x3", make_cfg(**base, dot_mode="bf16x3", solve_dot_mode="bf16x3", b3_dot_mode="bf16x3")),
                      ("default", make_cfg(**base, dot_mode="default", solve_dot_mode="default", b3_dot_mode="default")),
                      ("prod_mix_bt64", make_cfg(**base)),
                      ("make_cfg_bt128", make_cfg())):
        fn = make_blr_trainable(cfg, scale)

        def step():
            o, hf = fn(*xs)
            return torch.autograd.grad((o, hf), xs, grad_outputs=(2.0 * o, 2.0 * hf))

        ms = _median_ms(step)
        _lib.prof_begin(4 * 16)
        for _ in range(4):
            step()
        torch.cuda.synchronize()
        prof = _lib.prof_end()
        rows[name] = {"ms": round(ms, 4), "kernel_us": {n: round(t / c * 1e3, 1) for n, (t, c) in prof.items() if c}}
    return rows


def bench_config4(cfg, seed):
    """Config 4: forward-only long context, B8 H16 D128, bf16 inputs, fp32
    state; L = 32768 as 8 calls of 4096 tokens, each call's h0 = the previous h_final.  Inputs
    are drawn on the device (same distributions) per call."""
    import torch
    from atomic_gdn2 import make_blr_trainable, _lib
    from atomic_gdn2.synthetic import make_inputs_device
    B, H, D, Lc, ncall = 8, 16, 128, 4096, 8
    calls = [make_inputs_device(B, H, Lc, D, seed=seed * 100 + c, dtype=torch.bfloat16)[0] for c in range(ncall)]
    fn = make_blr_trainable(cfg, D ** -0.5)

    def run():
        h = None
        with torch.no_grad():
            for xs in calls:
                o, h = fn(*xs, h)
        return o, h

    ms = _median_ms(run, reps=2, rounds=3, warm=1)
    _lib.prof_begin(ncall * 4)
    run()
    torch.cuda.synchronize()
    prof = _lib.prof_end()
    N = B * H * Lc * ncall * D
    S = B * H * D * D * 4
    byts = 6 * N * 2 + N * 4 + 16 * S
    flops = B * H * Lc * ncall * (10 * 64 * D + 6 * D * D)
    kern = {n: round(t / c, 4) for n, (t, c) in prof.items() if c}
    return {"B": B, "H": H, "L": Lc * ncall, "D": D, "calls": ncall, "input_dtype": "bf16", "ms": round(ms, 3),
            "tokens_per_s": round(B * Lc * ncall / (ms * 1e-3), 1),
            "canonical_gb_per_s": round(byts / (ms * 1e-3) / 1e9, 1),
            "tflops": round(flops / (ms * 1e-3) / 1e12, 2), "kernel_ms_per_call": kern}


def bench_inference(cfg, seed):
    """The inference entry points (atomic_gdn2.inference, the reference's INFERENCE_V031) at
    config 4's serving shape B8 H16 D128: decode_step (one token, state read and written once,
    no MFMA) with fp32 and with bfloat16 inputs / state, and at B64 (fp32), and the prefill
    chunk_forward_inference of one config-4 call (L 4096, bf16 inputs) with four chunk-aligned
    documents per row, beside the same call without documents through make_blr_trainable.
    kernel_us / hbm_gb_per_s: HIP events around the decode kernel; ms: wall time per call,
    host work included (the prefill's domain and boundary checks synchronise with the device)."""
    import torch
    from atomic_gdn2 import make_blr_trainable, _lib
    from atomic_gdn2.inference import decode_step, chunk_forward_inference
    from atomic_gdn2.synthetic import make_inputs_device
    B, H, D = 8, 16, 128
    out = {"B": B, "H": H, "D": D}
    xs, scale = make_inputs_device(B, H, 1, D, seed=seed)
    x1 = [x[:, :, 0].contiguous() for x in xs]
    big, _ = make_inputs_device(64, H, 1, D, seed=seed)
    x64 = [x[:, :, 0].contiguous() for x in big]
    for name, dt, xb in (("decode_fp32", torch.float32, x1), ("decode_bf16", torch.bfloat16, x1),
                         ("decode_fp32_B64", torch.float32, x64)):
        Bn = xb[0].shape[0]
        xi = [x.to(dt) for x in xb]
        st = torch.zeros(Bn, H, D, D, device="cuda", dtype=dt)

        def run():
            decode_step(*xi, st, scale, state_dtype=dt)
        ms = _median_ms(run, reps=20, rounds=3, warm=3)
        _lib.prof_begin(64)
        for _ in range(20):
            run()
        torch.cuda.synchronize()
        t, c = _lib.prof_end()["decode"]
        us = t / c * 1e3
        eb = 2 if dt == torch.bfloat16 else 4
        byts = 2 * Bn * H * D * D * eb + 7 * Bn * H * D * eb
        out[name] = {"B": Bn, "ms_per_call": round(ms, 4), "kernel_us": round(us, 2), "bytes": byts,
                     "hbm_gb_per_s": round(byts / (us * 1e-6) / 1e9, 1),
                     "hbm_frac": round(byts / (us * 1e-6) / 1e9 / PEAK_HBM, 3)}
    L = 4096
    xs, scale = make_inputs_device(B, H, L, D, seed=seed + 1, dtype=torch.bfloat16)
    ids = torch.zeros(B, L, dtype=torch.int64, device="cuda")
    for s0 in (1024, 2048, 3072):
        ids[:, s0:] += 1
    fn = make_blr_trainable(cfg, scale)

    def plain():
        with torch.no_grad():
            fn(*xs)

    def docs():
        chunk_forward_inference(*xs, scale, cfg, segment_ids=ids)
    out["prefill_4_documents"] = {"L": L, "input_dtype": "bf16",
                                  "ms": round(_median_ms(docs, reps=2, rounds=3, warm=1), 3),
                                  "forward_only_ms": round(_median_ms(plain, reps=2, rounds=3, warm=1), 3)}
    return out


def hbm_stream_rates(n_bytes=1 << 30, reps=10):
    """The box's HBM streaming rates (TB/s): copy (bytes read + written), read and fill, by the
    library's one-float4-per-thread probe (gdn2_debug_stream), timed with HIP events on the
    stream it runs on; the median of 3 rounds of `reps` launches after 3 untimed ones."""
    import torch
    from atomic_gdn2 import _lib
    src = torch.ones(n_bytes // 4, device="cuda")
    dst = torch.empty_like(src)
    L_ = _lib.lib()
    stream = _lib.stream_handle(src.device)
    out = {}
    for mode, name, moved in ((0, "copy", 2 * n_bytes), (1, "read", n_bytes), (2, "fill", n_bytes)):
        def run():
            _lib.check(L_.gdn2_debug_stream(mode, _lib.ptr(src), _lib.ptr(dst), n_bytes, stream),
                       "gdn2_debug_stream")
        for _ in range(3):
            run()
        per = []
        for _ in range(3):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()                              # torch's current stream = the launch stream
            for _ in range(reps):
                run()
            e1.record()
            e1.synchronize()
            per.append(e0.elapsed_time(e1) / reps)
        ms = sorted(per)[1]
        out[name] = round(moved / (ms * 1e-3) / 1e12, 3)
    del src, dst
    torch.cuda.empty_cache()
    return out


def mfma_sustained_rates(iters=5120):
    """The box's sustained fp32 MFMA rate (TFLOP/s) with one and with two waves per SIMD: the
    library's probe (gdn2_debug_mfma: eight independent 16-deep mma16 products per round) on
    one (two) four-wave workgroups per CU, timed with HIP events on its stream; the median of 3
    launches after one untimed one.  A context figure for the kernels' MFMA rates: the roofline
    keeps the published peak."""
    import torch
    from atomic_gdn2 import _lib
    n_cu = torch.cuda.get_device_properties(0).multi_processor_count
    L_ = _lib.lib()
    stream = _lib.stream_handle()
    out = {}
    for wps in (1, 2):
        blocks = n_cu * wps
        buf = torch.empty(blocks * 256, device="cuda")

        def run():
            _lib.check(L_.gdn2_debug_mfma(blocks, iters, _lib.ptr(buf), stream), "gdn2_debug_mfma")
        run()
        per = []
        for _ in range(3):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()                              # torch's current stream = the launch stream
            run()
            e1.record()
            e1.synchronize()
            per.append(e0.elapsed_time(e1))
        ms = sorted(per)[1]
        flop = blocks * 4 * iters * 8 * 8192
        out[f"waves_per_simd_{wps}"] = round(flop / (ms * 1e-3) / 1e12, 1)
    out["published_peak"] = PEAK_FP32_MFMA
    return out


def bench_e2e_lm(seed, reps=4, rounds=3, warm=2):
    """Config 5: one training step of the reference's benchmark LM (8 GDN-2
    blocks, 34,873,952 parameters, B8 L2048, vocab 256, CE + clip_by_global_norm(1.0) + AdamW)
    on uniform synthetic tokens, the optimizer state evolving across the timed steps as in the
    reference's protocol (candidate_e2e.py timed_step)."""
    import torch
    from atomic_gdn2 import e2e_lm
    torch.backends.cuda.matmul.allow_tf32 = False
    cfg = e2e_lm.LMConfig()
    model = e2e_lm.make_lm(cfg, seed=seed)
    step = e2e_lm.TrainStep(model)
    ids = e2e_lm.synthetic_tokens(cfg, batch=8, length=2048, seed=seed)
    loss = [None]

    def run():
        loss[0] = step(ids)

    ms = _median_ms(run, reps=reps, rounds=rounds, warm=warm)
    final = float(loss[0])
    return {"params": e2e_lm.n_params(model), "batch": 8, "length": 2048, "ms_per_step": round(ms, 3),
            "input_tokens_per_s": round(8 * 2048 / (ms * 1e-3), 1), "final_loss": round(final, 4),
            "finite": bool(math.isfinite(final)), "operator_cfg": "bt64 wy_eps0 (the reference's no_damping speed profile) dot=highest",
            "matmul": "fp32", "reference_tpu_v5e_ms": 204.659}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--state-ckpt", type=int, default=None,
                    help="residual state checkpoint interval K (0 = every chunk's state kept); "
                         "default: the library's DEFAULT_STATE_CKPT")
    ap.add_argument("--ckpt-table", action="store_true", help="only print the state_ckpt table and exit")
    ap.add_argument("--dot-table", action="store_true", help="only print the dot-mode table and exit")
    ap.add_argument("--inference", action="store_true", help="only print the inference entry points' figures and exit")
    ap.add_argument("--profile-only", action="store_true",
                    help="for rocprofv3: run --warmup then --steps gradient evaluations of the workload "
                         "(no timing loops, no forward-only pass, no other configs) and print nothing else")
    ap.add_argument("--seq-len", type=int, default=L_,
                    help="sequence length of the workload for --profile-only (default 2048, config 2)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-sweep", action="store_true", help="skip the config-3 sweep and the config-4 run")
    ap.add_argument("--no-e2e", action="store_true", help="skip the end-to-end LM training step")
    ap.add_argument("--hbm-rates", action="store_true",
                    help="only print the HBM copy / read / fill rates of the streaming probe and exit")
    ap.add_argument("--mfma-rate", action="store_true",
                    help="only print the sustained fp32 MFMA rates (gdn2_debug_mfma) and exit")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run 5 plain device copies of a 256 MiB fp32 buffer (reference for the "
                         "FETCH_SIZE / WRITE_SIZE counters) and exit")
    args = ap.parse_args()
    if args.calibrate_copy:
        import torch
        src = torch.ones(64 * 2 ** 20, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": src.numel() * 4, "copy_bytes_written": dst.numel() * 4, "copies": 5}))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: every (batch, head) sequence is independent, so a "
              "multi-GPU run is B/H sharding with no communication; run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)

    import torch
    from atomic_gdn2 import make_cfg, make_blr_trainable, _lib
    from atomic_gdn2.synthetic import make_inputs, make_inputs_np, inputs_sha256

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    arrs, scale = make_inputs_np(B_, H_, L_, D_, seed=args.seed)
    sha = inputs_sha256(arrs)                      # recorded as the reference harness does
    q, k, v, w, b, g = (torch.from_numpy(x).to(dev) for x in arrs)
    del arrs
    xs = [t.requires_grad_(True) for t in (q, k, v, w, b, g)]
    cfg = make_cfg(bt=64, bc=32, score_bs=64, bs2=32, mb=8, wy_eps=0.0, dot_mode="highest",
                   solve_dot_mode="highest", b3_dot_mode="highest")
    from atomic_gdn2.pipeline import DEFAULT_STATE_CKPT
    ckpt = DEFAULT_STATE_CKPT if args.state_ckpt is None else args.state_ckpt
    if args.ckpt_table:
        print(json.dumps({"state_ckpt_table": state_ckpt_table(cfg, args.seed)}), flush=True)
        return
    if args.dot_table:
        print(json.dumps({"dot_mode_ms": dot_mode_table(args.seed)}), flush=True)
        return
    if args.inference:
        print(json.dumps({"inference": bench_inference(cfg, args.seed)}), flush=True)
        return
    if args.hbm_rates:
        print(json.dumps({"hbm_stream_tb_s": hbm_stream_rates()}), flush=True)
        return
    if args.mfma_rate:
        print(json.dumps({"mfma_fp32_sustained_tflops": mfma_sustained_rates()}), flush=True)
        return
    if args.profile_only:
        if args.seq_len == L_:
            pxs, pscale = xs, scale
        else:
            pts, pscale = make_inputs(B_, H_, args.seq_len, D_, seed=args.seed)
            pxs = [t.requires_grad_(True) for t in pts]
        pfn = make_blr_trainable(cfg, pscale, state_ckpt=ckpt)
        for _ in range(args.warmup + args.steps):
            o, hf = pfn(*pxs)
            torch.autograd.grad((o, hf), pxs, grad_outputs=(2.0 * o, 2.0 * hf))
        torch.cuda.synchronize()
        print(json.dumps({"profile_only": True, "B": B_, "H": H_, "L": args.seq_len, "state_ckpt": ckpt,
                          "grad_evals": args.warmup + args.steps}), flush=True)
        return
    fn = make_blr_trainable(cfg, scale, state_ckpt=ckpt)

    def step():
        # gradient of loss = sum(o^2) + sum(h_final^2): forward, the loss's cotangents
        # d loss/d o = 2 o and d loss/d h_final = 2 h_final, and the operator's VJP.  Like
        # jax.grad of the same loss, the step returns the gradients only (the scalar loss value
        # feeds nothing and is not formed).
        o, hf = fn(*xs)
        return torch.autograd.grad((o, hf), xs, grad_outputs=(2.0 * o, 2.0 * hf))

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ms = dt * 1e3 / args.steps
    # per-kernel durations: a separate pass with HIP events around every library launch
    # (the events add gaps of their own, so the timed loop above runs without them)
    _lib.prof_begin(args.steps * len(_lib.KERNEL_NAMES) + 16)
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    prof = _lib.prof_end()

    # forward-only (no residuals) throughput on the same inputs
    with torch.no_grad():
        for _ in range(2):
            fn(q.detach(), k.detach(), v.detach(), w.detach(), b.detach(), g.detach())
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        for _ in range(args.steps):
            fn(q.detach(), k.detach(), v.detach(), w.detach(), b.detach(), g.detach())
        torch.cuda.synchronize()
        fwd_ms = (time.perf_counter() - t1) * 1e3 / args.steps

    ff, fb = canonical_flops(B_, H_, L_, D_)
    tflops = (ff + fb) / (ms * 1e-3) / 1e12
    kf = kernel_flops_per_token(fused_out=ckpt > 0)
    ntok = B_ * H_ * L_
    # HBM bytes per launch measured by rocprof counters (FETCH_SIZE / WRITE_SIZE, scaled by a
    # copy kernel) at this workload; with this launch's own time they give each kernel's
    # achieved HBM bandwidth (the bound the sequential scans are reported against).
    tf = ROOT / "profiles" / "traffic.json"
    tmeas = json.loads(tf.read_text()) if tf.exists() else {}
    kern = {}
    for name, (tot_ms, cnt) in prof.items():
        if cnt:
            avg = tot_ms / cnt
            kern[name] = {"avg_ms": round(avg, 5), "launches": cnt,
                          "tflops": round(kf[name] * ntok / (avg * 1e-3) / 1e12, 2)}
            if isinstance(tmeas.get(name), int):
                kern[name]["hbm_gb_per_s"] = round(tmeas[name] / (avg * 1e-3) / 1e9, 1)
    dom = max(kern, key=lambda n: kern[n]["avg_ms"])
    ach = kern[dom]["tflops"]
    traffic = tmeas.get(dom)

    out = {
        "metric": "fwd+bwd ms, TFLOP/s and MFMA % at B4 H6 L2048 D128 fp32; fwd tokens/s",
        "value": round(tflops, 3), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp32", "data": "synthetic",
        "config": {"workload": "gdn2 grad-eval (fwd+bwd of sum(o^2)+sum(h_final^2)) B4 H6 L2048 D128 "
                               "chunk64 wy_eps0 dot=highest", "B": B_, "H": H_, "L": L_, "D": D_, "bt": 64,
                   "seed": args.seed, "inputs_sha256": sha, "state_ckpt": ckpt},
        "fwd_ms": round(fwd_ms, 4), "fwd_tokens_per_s": round(B_ * L_ / (fwd_ms * 1e-3), 1),
        "canonical_gflop": round((ff + fb) / 1e9, 3),
        "canonical_gb_per_s": round(canonical_bytes(B_, H_, L_, D_) / (ms * 1e-3) / 1e9, 1),
        "mfma_frac_of_fp32_peak_step": round(tflops / PEAK_FP32_MFMA, 4),
        "kernels": kern,
        "roofline": {"kernel": dom, "bound": "mfma", "achieved": ach, "peak": PEAK_FP32_MFMA,
                     "unit": "TFLOP/s", "frac": round(ach / PEAK_FP32_MFMA, 4), "traffic": traffic},
        "reference_tpu_v5e_ms": 2.888,
    }
    # each kernel's achieved HBM rate against what a plain copy reaches on this box
    rates = hbm_stream_rates()
    out["hbm_stream_tb_s"] = rates
    out["mfma_fp32_sustained_tflops"] = mfma_sustained_rates()
    for kd in kern.values():
        if "hbm_gb_per_s" in kd:
            kd["hbm_frac_of_copy"] = round(kd["hbm_gb_per_s"] / 1e3 / rates["copy"], 3)
    t_start = time.perf_counter()

    def section(name, fn):
        # one progress line per section on stderr (the JSON line on stdout stays the only output there)
        r = fn()
        print(f"[bench] {name} done at {time.perf_counter() - t_start:.0f} s", file=sys.stderr, flush=True)
        return r

    print(f"[bench] config 2: {ms:.4f} ms per grad-eval", file=sys.stderr, flush=True)
    if not args.no_sweep:
        out["config2_seeds"] = section("config2 seeds", lambda: seeds_config2(cfg))
        out["state_ckpt_table"] = section("state_ckpt table", lambda: state_ckpt_table(cfg, args.seed))
        out["dot_mode_ms"] = section("dot modes", lambda: dot_mode_table(args.seed))
        out["config3_sweep"] = section("config3 sweep", lambda: sweep_config3(cfg, args.seed))
        out["config4_long_context_fwd"] = section("config4", lambda: bench_config4(cfg, args.seed))
        out["inference"] = section("inference", lambda: bench_inference(cfg, args.seed))
    if not args.no_e2e:
        out["config5_e2e_lm"] = section("config5 e2e LM", lambda: bench_e2e_lm(args.seed))
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = section("cpu baseline", cpu_baseline)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
