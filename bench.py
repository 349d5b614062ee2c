#!/usr/bin/env python3
"""Benchmark of the Nova GPU matmul / reduction path on one MI355X.

One step = one launch of the hot path over one batch of synthetic input,
inputs already resident in HBM.  The headline (``value``) is config 2 of
linalg.batch_matmul bf16 -> f32, B=8, M=N=K=4096, in TFLOP/s.
The same line carries configs 3-5 (linear+bias+GELU, the unaligned fp16
batch GEMMs, LayerNorm and softmax cross-entropy) as ``configs``, each with
its roofline fraction, the ``roofline`` object of the dominant kernel, and a
``cpu_baseline`` timed on this host with the CPU oracle.

Timing: torch.cuda.Event pairs on torch's current stream, which is the
stream libnova_hip launches on (nova_hip.py binds it before every call).
Each timed pass of back-to-back launches follows the --warmup calls and as
many more untimed ones as make up 0.2 s of work (MIN_WARM_MS), so that it
measures the clock the board settles at under sustained load.  Inputs of
every config whose working set is under 1 GB rotate over 3 buffer sets so
the 256 MB MALL cannot serve repeated reads as if they were HBM traffic.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "nova-compiler_amd"))

# MI355X published peaks (dense).
PEAK_BF16_TFLOPS = 2516.6   # 256 CU x 2.4 GHz x 4096 FLOP/clk/CU
PEAK_HBM_GBS = 8000.0

C1_FLOP = 2 * 256 ** 3                       # 33,554,432
C2_FLOP = 2 * 8 * 4096 ** 3                  # 1,099,511,627,776
C3_FLOP = 2 * 4096 * 4096 * 11008            # 369,367,187,456
C4_FLOP = 2 * 96 * 197 * 197 * 64            # 476,884,992 (both shapes)
C4A_BYTES = 19_744_128
C4B_BYTES = 14_713_536
LN_BYTES = 16384 * 4096 * 4 * 2 + 4096 * 4 * 2 + 16384 * 4 * 2   # 537,034,752
SCE_BYTES = 4096 * 32000 * 4 + 4096 * 4 + 4                     # 524,304,388
# Backward ops at the same config-5 / config-3 shapes (algorithmic bytes /
# FLOP; workspace partials excluded).
SCE_BWD_BYTES = 2 * 4096 * 32000 * 4 + 4096 * 4                 # 1,048,592,384
SCE_FWD_BWD_BYTES = 2 * 4096 * 32000 * 4 + 4096 * 4 + 4         # 1,048,592,388
LN_BWD_BYTES = 3 * 16384 * 4096 * 4 + 4096 * 4 * 3 + 16384 * 4 * 2  # 805,486,592
C3_BWD_FLOP = 2 * C3_FLOP                                       # grad_input + grad_weight


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true",
                    help="skip the CPU oracle timing (cpu_baseline becomes null)")
    ap.add_argument("--telemetry", action="store_true",
                    help="also run config 2 (this library and hipBLASLt), config 3 and an MFMA-only probe "
                         "back to back for --telemetry-seconds each while sampling board power "
                         "and clocks with amd-smi (reported under 'telemetry')")
    ap.add_argument("--telemetry-seconds", type=float, default=6.0)
    ap.add_argument("--only", default="",
                    help="comma list of configs to run (c2,c3,c4,ln,sce,sce_bwd,sce_fwd_bwd,ln_bwd,"
                         "c3_bwd,c2_vendor,gpt_step; copy = HBM copy calibration); the HBM "
                         "copy ceiling runs whenever a reduction config does")
    return ap.parse_args()


def to_dev(a, dt, torch):
    import numpy as np
    import nova_seed as S
    if dt == S.F32:
        return torch.from_numpy(np.ascontiguousarray(a)).cuda()
    t = torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda()
    return t.view(torch.bfloat16 if dt == S.BF16 else torch.float16)


# Per-launch distribution of the last time_launches call (see there).
_LAUNCH_STATS = {}


# Untimed back-to-back work before each timed pass, at least (ms): the first
# tens of milliseconds after a stage starts run slow while the clock settles
# under the board's power limit (config 3: 25 launches after 5 warm-up calls
# measured 0.384 ms per launch, 200 launches after 0.2 s of warm-up 0.325 ms,
# on one box).
MIN_WARM_MS = 200.0


def time_launches(fn, steps, warmup, torch):
    """Average ms per call over `steps` back-to-back calls (the returned
    figure), after `warmup` calls and then as many more untimed calls as
    make up MIN_WARM_MS of back-to-back work.  A second pass of `steps`
    calls, each between two events, gives the median and p10 / p90 of
    single launches in _LAUNCH_STATS; those events add a little to each
    launch, so the average is taken from the first pass only."""
    w0 = torch.cuda.Event(enable_timing=True)
    w1 = torch.cuda.Event(enable_timing=True)
    done, n, batch = 0.0, 0, max(warmup, 1)
    while n < warmup or done < MIN_WARM_MS:
        w0.record()
        for i in range(batch):
            fn(n + i)
        w1.record()
        torch.cuda.synchronize()
        done += w0.elapsed_time(w1)
        n += batch
        per = done / n
        batch = max(1, min(10000, int((MIN_WARM_MS - done) / max(per, 1e-3)) + 1))
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        fn(i)
    end.record()
    torch.cuda.synchronize()
    avg = start.elapsed_time(end) / steps
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    ev[0].record()
    for i in range(steps):
        fn(i)
        ev[i + 1].record()
    torch.cuda.synchronize()
    t = sorted(ev[i].elapsed_time(ev[i + 1]) for i in range(steps))

    def q(f):
        return t[min(len(t) - 1, int(round(f * (len(t) - 1))))]

    _LAUNCH_STATS.clear()
    _LAUNCH_STATS.update({"p10": q(0.1), "p50": q(0.5), "p90": q(0.9), "n": steps})
    return avg


def bench_c2(args, torch, nh, S):
    inp = S.config_inputs("c2")
    A = to_dev(inp["A"], S.BF16, torch)
    B = to_dev(inp["B"], S.BF16, torch)
    del inp
    C = torch.empty(8, 4096, 4096, device="cuda", dtype=torch.float32)
    dA, dB, dC = nh.memref_of(A), nh.memref_of(B), nh.memref_of(C)
    L = nh.lib()
    fn_ = L._mlir_ciface_nova_hip_batch_matmul_bf16_f32
    pA, pB, pC = nh.ref(dA), nh.ref(dB), nh.ref(dC)

    def fn(_):
        rc = fn_(pA, pB, pC)
        if rc:
            nh.check(rc)

    nh._bind_stream()
    ms = time_launches(fn, args.steps, args.warmup, torch)
    finite = bool(torch.isfinite(C[:, ::512, ::512]).all())
    del A, B, C
    tf = C2_FLOP / (ms * 1e-3) / 1e12
    return {"ms": ms, "tflops": tf, "frac_mfma": tf / PEAK_BF16_TFLOPS, "finite": finite}


def bench_c1(args, torch, nh, S):
    """Config 1, the plumbing case: nova.matmul f32 256x256 . 256x256 on the
    exact f32 kernel (bit-identical to the CPU pipeline)."""
    inp = S.config_inputs("c1")
    A, B = to_dev(inp["A"], S.F32, torch), to_dev(inp["B"], S.F32, torch)
    C = torch.empty(256, 256, device="cuda")
    d = [nh.ref(nh.memref_of(t)) for t in (A, B, C)]
    f_ = nh.lib()._mlir_ciface_nova_hip_matmul_f32

    def fn(_):
        rc = f_(*d)
        if rc:
            nh.check(rc)

    nh._bind_stream()
    ms = time_launches(fn, args.steps * 4, args.warmup, torch)
    return {"ms": ms, "tflops": C1_FLOP / (ms * 1e-3) / 1e12}


def bench_c3(args, torch, nh, S):
    """Config 3 over three rotated buffer sets (3 x 204 MB, more than the
    256 MB MALL holds), so no launch finds its operands in the cache the
    previous one filled."""
    inp = S.config_inputs("c3")
    sets = []
    for _ in range(3):
        x = to_dev(inp["x"], S.BF16, torch)
        W = to_dev(inp["W"], S.BF16, torch)
        b = to_dev(inp["bias"], S.BF16, torch)
        y = torch.empty(4096, 11008, device="cuda", dtype=torch.bfloat16)
        d = [nh.memref_of(t) for t in (x, W.t(), b, y)]
        sets.append(([nh.ref(v) for v in d], (x, W, b, y, d)))
    del inp
    f_ = nh.lib()._mlir_ciface_nova_hip_linear_bf16_bias_gelu

    def fn(i):
        rc = f_(*sets[i % 3][0])
        if rc:
            nh.check(rc)

    nh._bind_stream()
    ms = time_launches(fn, max(args.steps // 2, 5), max(args.warmup // 2, 2), torch)
    tf = C3_FLOP / (ms * 1e-3) / 1e12
    return {"ms": ms, "tflops": tf, "frac_mfma": tf / PEAK_BF16_TFLOPS}


def bench_c4(args, torch, nh, S, name, nbytes):
    inp = S.config_inputs(name)
    sets = []
    for _ in range(3):
        A = to_dev(inp["A"], S.F16, torch)
        B = to_dev(inp["B"], S.F16, torch)
        C = torch.empty(A.shape[0], A.shape[1], B.shape[2], device="cuda")
        sets.append(tuple(nh.ref(nh.memref_of(t)) for t in (A, B, C)) + (A, B, C))
    f_ = nh.lib()._mlir_ciface_nova_hip_batch_matmul_f16_f32

    def fn(i):
        s = sets[i % 3]
        rc = f_(s[0], s[1], s[2])
        if rc:
            nh.check(rc)

    nh._bind_stream()
    ms = time_launches(fn, args.steps * 4, args.warmup, torch)
    tf = C4_FLOP / (ms * 1e-3) / 1e12
    gbs = nbytes / (ms * 1e-3) / 1e9
    # binding roof: min(MFMA peak, AI x HBM)
    roof = min(PEAK_BF16_TFLOPS, (C4_FLOP / nbytes) * PEAK_HBM_GBS / 1e3)
    return {"ms": ms, "tflops": tf, "gbs": gbs, "roof_tflops": roof, "frac_roof": tf / roof}


def bench_ln(args, torch, nh, S):
    inp = S.config_inputs("c5_ln")
    g = to_dev(inp["gamma"], S.F32, torch)
    b = to_dev(inp["beta"], S.F32, torch)
    sets = []
    for _ in range(3):
        x = to_dev(inp["x"], S.F32, torch)
        y = torch.empty_like(x)
        s = torch.empty(16384, device="cuda")
        r = torch.empty(16384, device="cuda")
        sets.append(([nh.ref(nh.memref_of(t)) for t in (x, g, b, y, s, r)], (x, y, s, r)))
    del inp
    import ctypes
    f_ = nh.lib()._mlir_ciface_nova_hip_layer_norm_f32
    eps = ctypes.c_float(1e-5)

    def fn(i):
        p = sets[i % 3][0]
        rc = f_(*p, eps)
        if rc:
            nh.check(rc)

    nh._bind_stream()
    ms = time_launches(fn, args.steps * 2, args.warmup, torch)
    gbs = LN_BYTES / (ms * 1e-3) / 1e9
    return {"ms": ms, "gbs": gbs, "frac_hbm": gbs / PEAK_HBM_GBS}


def bench_sce(args, torch, nh, S):
    inp = S.config_inputs("c5_sce")
    sets = []
    for _ in range(3):
        x = to_dev(inp["logits"], S.F32, torch)
        t = torch.from_numpy(inp["labels"]).cuda()
        loss = torch.empty(1, device="cuda")
        sets.append(([nh.ref(nh.memref_of(v)) for v in (x, t, loss)], (x, t, loss)))
    del inp
    f_ = nh.lib()._mlir_ciface_nova_hip_sce_f32

    def fn(i):
        p = sets[i % 3][0]
        rc = f_(p[0], p[1], p[2], None)
        if rc:
            nh.check(rc)

    nh._bind_stream()
    ms = time_launches(fn, args.steps * 2, args.warmup, torch)
    gbs = SCE_BYTES / (ms * 1e-3) / 1e9
    return {"ms": ms, "gbs": gbs, "frac_hbm": gbs / PEAK_HBM_GBS,
            "loss": float(sets[0][1][2].cpu()[0])}


def bench_sce_bwd(args, torch, nh, S, fused):
    """nova.sce_backward on the config-5 SCE shape (softmax in, grad out),
    or the fused forward + backward (logits in, loss and grad out)."""
    inp = S.config_inputs("c5_sce")
    sets = []
    for _ in range(3):
        x = to_dev(inp["logits"], S.F32, torch)
        t = torch.from_numpy(inp["labels"]).cuda()
        g = torch.empty_like(x)
        loss = torch.empty(1, device="cuda")
        d = (x, t, loss, g) if fused else (x, t, g)
        sets.append(([nh.ref(nh.memref_of(v)) for v in d], d))
    del inp
    f_ = (nh.lib()._mlir_ciface_nova_hip_sce_fwd_bwd_f32 if fused
          else nh.lib()._mlir_ciface_nova_hip_sce_backward_f32)

    def fn(i):
        rc = f_(*sets[i % 3][0])
        if rc:
            nh.check(rc)

    nh._bind_stream()
    ms = time_launches(fn, args.steps * 2, args.warmup, torch)
    nbytes = SCE_FWD_BWD_BYTES if fused else SCE_BWD_BYTES
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"ms": ms, "gbs": gbs, "frac_hbm": gbs / PEAK_HBM_GBS, "bytes": nbytes}


def bench_ln_bwd(args, torch, nh, S):
    """nova.layer_norm_backward on the config-5 LayerNorm shape."""
    inp = S.config_inputs("c5_ln")
    g = to_dev(inp["gamma"], S.F32, torch)
    x0 = to_dev(inp["x"], S.F32, torch)
    y, Sm, rs = nh.layer_norm(x0, g, to_dev(inp["beta"], S.F32, torch))
    del y
    sets = []
    for i in range(3):
        x = x0 if i == 0 else x0.clone()
        gy = torch.randn_like(x0)
        dx = torch.empty_like(x0)
        dg = torch.empty(4096, device="cuda")
        db = torch.empty(4096, device="cuda")
        d = (gy, x, g, Sm, rs, dx, dg, db)
        sets.append(([nh.ref(nh.memref_of(v)) for v in d], d))
    del inp
    f_ = nh.lib()._mlir_ciface_nova_hip_layer_norm_backward_f32

    def fn(i):
        rc = f_(*sets[i % 3][0])
        if rc:
            nh.check(rc)

    nh._bind_stream()
    ms = time_launches(fn, args.steps * 2, args.warmup, torch)
    gbs = LN_BWD_BYTES / (ms * 1e-3) / 1e9
    return {"ms": ms, "gbs": gbs, "frac_hbm": gbs / PEAK_HBM_GBS, "bytes": LN_BWD_BYTES}


def bench_c3_bwd(args, torch, nh, S):
    """nova.linear_backward of config 3 (bf16 in, f32 accumulate, f32
    grads): grad_input = go . W, grad_weight written in W's [11008, 4096]
    layout, grad_bias; TFLOP/s over the two GEMMs."""
    inp = S.config_inputs("c3")
    sets = []
    for _ in range(3):   # rotated: 3 x 537 MB
        x = to_dev(inp["x"], S.BF16, torch)
        W = to_dev(inp["W"], S.BF16, torch)
        go = torch.randn(4096, 11008, device="cuda").to(torch.bfloat16)
        gi = torch.empty(4096, 4096, device="cuda")
        gw = torch.empty(11008, 4096, device="cuda")
        gb = torch.empty(11008, device="cuda")
        d = [nh.memref_of(t) for t in (go, x, W.t(), gi, gw.t(), gb)]
        sets.append(([nh.ref(v) for v in d], (x, W, go, gi, gw, gb, d)))
    del inp
    flags = nh.gemm_flags(nh.DT_BF16, nh.DT_F32)
    f_ = nh.lib()._mlir_ciface_nova_hip_linear_backward

    def fn(i):
        rc = f_(*sets[i % 3][0], flags)
        if rc:
            nh.check(rc)

    nh._bind_stream()
    ms = time_launches(fn, max(args.steps // 2, 5), max(args.warmup // 2, 2), torch)
    tf = C3_BWD_FLOP / (ms * 1e-3) / 1e12
    return {"ms": ms, "tflops": tf, "frac_mfma": tf / PEAK_BF16_TFLOPS}


def bench_c2_vendor(args, torch, S):
    """The vendor library on config 2 for comparison, not part of this
    build: torch.bmm (hipBLASLt on ROCm) with bf16 inputs and f32 output,
    the same inputs and timing as bench_c2."""
    inp = S.config_inputs("c2")
    A = to_dev(inp["A"], S.BF16, torch)
    B = to_dev(inp["B"], S.BF16, torch)
    del inp
    C = torch.empty(8, 4096, 4096, device="cuda", dtype=torch.float32)

    def fn(_):
        torch.bmm(A, B, out_dtype=torch.float32, out=C)

    try:
        ms = time_launches(fn, args.steps, args.warmup, torch)
    except (TypeError, RuntimeError) as e:  # torch without out_dtype support
        return {"error": str(e)[:200]}
    tf = C2_FLOP / (ms * 1e-3) / 1e12
    return {"ms": ms, "tflops": tf, "frac_mfma": tf / PEAK_BF16_TFLOPS,
            "library": "torch.bmm(out_dtype=float32) -> hipBLASLt"}


def bench_copy(args, torch):
    """A plain device copy of 256 MiB (torch's copy kernel): the practical
    read+write HBM ceiling the reductions are compared with, and the known
    byte count that calibrates the FETCH_SIZE / WRITE_SIZE counters."""
    n = 64 * 1024 * 1024
    xs = [torch.empty(n, device="cuda").fill_(1.0) for _ in range(3)]
    ys = [torch.empty(n, device="cuda") for _ in range(3)]

    def fn(i):
        ys[i % 3].copy_(xs[i % 3])

    ms = time_launches(fn, args.steps * 2, args.warmup, torch)
    gbs = 2 * n * 4 / (ms * 1e-3) / 1e9
    return {"ms": ms, "bytes": 2 * n * 4, "gbs": gbs, "frac_hbm": gbs / PEAK_HBM_GBS}


def bench_copy_ceiling(args, torch):
    """The practical HBM read+write ceiling on this box: the fastest copy
    form (nova-compiler_amd/libnova_probe.so nova_probe_copy: one 16-byte
    element per thread, nontemporal) over 256 MiB, three rotated buffer
    sets.  The reductions' GB/s are also given as a fraction of it
    (frac_copy_ceiling), beside their fraction of the 8 TB/s peak."""
    import ctypes
    try:
        probe = ctypes.CDLL(os.path.join(REPO, "nova-compiler_amd", "libnova_probe.so"))
    except OSError as e:  # the probe library is a measurement aid, not the op path
        return {"error": f"libnova_probe.so not loaded: {e}"[:200]}
    probe.nova_probe_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                      ctypes.c_void_p]
    n = 64 * 1024 * 1024
    xs = [torch.empty(n, device="cuda").fill_(1.0) for _ in range(3)]
    ys = [torch.empty(n, device="cuda") for _ in range(3)]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def fn(i):
        rc = probe.nova_probe_copy(ctypes.c_void_p(xs[i % 3].data_ptr()),
                                   ctypes.c_void_p(ys[i % 3].data_ptr()), n * 4, stream)
        if rc:
            raise RuntimeError(f"nova_probe_copy failed: {rc}")

    ms = time_launches(fn, args.steps * 2, args.warmup, torch)
    if not torch.equal(ys[0], xs[0]):
        raise RuntimeError("nova_probe_copy: the copy differs from its source")
    gbs = 2 * n * 4 / (ms * 1e-3) / 1e9
    return {"ms": ms, "bytes": 2 * n * 4, "gbs": gbs, "frac_hbm": gbs / PEAK_HBM_GBS}


def bench_gpt_step(args, torch):
    """A whole GPT training step (the reference GPT step's shapes: batch 8,
    1024 tokens, vocab 50304, width 384, MLP 1536; forward, SCE loss and the
    full backward to the embedding gradients) through libnova_run.  Timed
    with arguments and results resident in device memory
    (nova_run_execute_device, the reference's address-space-1 contract),
    once with the f32 GEMMs exact (bit-identical to the CPU pipeline) and
    once on the f32 matrix cores (1e-4 bar); events around back-to-back
    steps on the stream the launches go to.  The host-array form
    (nova_run_execute, PCIe copies of ~0.25 GB included) is timed once for
    comparison.  Weights random (N(0, 0.02)), so the loss is near ln(vocab)."""
    import numpy as np
    import nova_run
    from gpt_program import gpt_step
    B, T, V, D, H = 8, 1024, 50304, 384, 1536
    r = np.random.default_rng(6)

    def f(*s, k=0.02):
        return r.standard_normal(s, dtype=np.float32) * np.float32(k)

    inp = [r.integers(0, V, (B, T)).astype(np.int16), r.integers(0, V, (B, T)).astype(np.int16),
           np.arange(T, dtype=np.int64).reshape(1, T), f(V, D), f(T, D), 1 + f(D), f(D), f(D, H),
           f(H), f(H, D), f(D), 1 + f(D), f(D), f(D, V)]
    p = nova_run.Program(gpt_step(B, T, V, D, H))
    dev = [torch.from_numpy(a).cuda() for a in inp]
    res = {"launches": None}
    for mode, name in ((nova_run.F32_GEMM_EXACT, "exact"), (nova_run.F32_GEMM_MFMA, "mfma")):
        p.set_f32_gemm(mode)
        res["launches"] = p.plan("gpt_step").count("_mlir_ciface_")
        out = p.run_device("gpt_step", *dev)        # untimed: allocates the intermediates
        torch.cuda.synchronize()
        reps = 5
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            p.run_device("gpt_step", *dev, results=out)
        e1.record()
        torch.cuda.synchronize()
        res[f"ms_per_step_device_{name}"] = e0.elapsed_time(e1) / reps
        res[f"loss_{name}"] = float(out[0][0].item())
        res[f"finite_{name}"] = bool(all(torch.isfinite(o).all().item() for o in out))
    p.set_f32_gemm(nova_run.F32_GEMM_MFMA)
    p.run("gpt_step", *inp)
    t0 = time.perf_counter()
    p.run("gpt_step", *inp)
    res["ms_wall_host_arrays_mfma"] = (time.perf_counter() - t0) * 1e3
    res["ln_vocab"] = float(np.log(V))
    res["note"] = ("device-resident arguments and results, events over back-to-back steps; "
                   "f32 program (the reference GPT step's dtype); ms_wall_host_arrays includes "
                   "the host<->device copies")
    return res


def cpu_baseline(S):
    """The CPU oracle (restatement of Nova's single-threaded CPU pipeline)
    on a bounded slab of config 2: batch 0, the first R rows, all 4096
    columns, K = 4096; R grows until ~12 s of CPU work.  TFLOP/s of the
    slab, which extrapolates linearly to the full config."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import nova_cpu_ref as ref
    n = 8 * 4096 * 4096
    A = S.uniform((1, 4096, 4096), 1, dtype=S.BF16)
    B = S.uniform((1, 4096, 4096), 1, dtype=S.BF16, offset=n)
    rows, spent = 0, 0.0
    step = 8
    while spent < 12.0 and rows < 256:
        t0 = time.perf_counter()
        ref.gemm(A[:, rows:rows + step], B, adt=S.BF16, bdt=S.BF16)
        spent += time.perf_counter() - t0
        rows += step
    flop = 2.0 * rows * 4096 * 4096
    tf = flop / spent / 1e12
    return {"value": tf, "unit": "TFLOP/s", "cores": 1, "kind": "port",
            "sample": f"config 2 slab: batch 0, rows 0-{rows - 1}, all 4096 columns, K=4096 "
                      f"({flop:.3g} FLOP in {spent:.1f} s, single thread, "
                      f"oracle/nova_cpu_ref.c i-j-k loop order); extrapolated linearly",
            "full_config_seconds_extrapolated": C2_FLOP / (tf * 1e12),
            "host_cpus": os.cpu_count(), "host_cpu_model": cpu_model()}


def cpu_baselines(S, only):
    """The CPU oracle (one thread, the reference CPU pipeline's loop orders)
    on configs 1, 3, 4 and 5: configs 1, 4a, 4b, LayerNorm and SCE in full;
    config 3 on a slab of its first 8 rows (all 11008 outputs, K = 4096, bias
    + GELU, bf16 out), extrapolated linearly.  Seconds per full config and
    the rate in the config's unit."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import nova_cpu_ref as ref
    out = {}

    def timed(f):
        t0 = time.perf_counter()
        f()
        return time.perf_counter() - t0

    if "c1" in only:
        inp = S.config_inputs("c1")
        t = timed(lambda: ref.gemm(inp["A"], inp["B"]))
        out["c1_matmul_f32_256"] = {"value": C1_FLOP / t / 1e9, "unit": "GFLOP/s", "cores": 1,
                                    "kind": "port", "sample": "config 1 in full",
                                    "seconds_full_config": t}
    if "c3" in only:
        inp = S.config_inputs("c3")
        rows = 8
        x = inp["x"][:rows]
        t = timed(lambda: ref.gemm(x, inp["W"].T, adt=S.BF16, bdt=S.BF16, bias=inp["bias"],
                                   biasdt=S.BF16, epilogue=ref.EPI_BIAS_GELU, cdt=S.BF16))
        flop = 2.0 * rows * 4096 * 11008
        out["c3_linear_bias_gelu_bf16"] = {
            "value": flop / t / 1e9, "unit": "GFLOP/s", "cores": 1, "kind": "port",
            "sample": f"config 3 slab: rows 0-{rows - 1} of x, all 11008 outputs, K=4096, "
                      f"bias+GELU, bf16 out ({flop:.3g} FLOP in {t:.2f} s); extrapolated linearly",
            "seconds_full_config": t * 4096 / rows, "extrapolated": True}
    if "c4" in only:
        for name, key in (("c4a", "c4a_fp16_96x197x197x64"), ("c4b", "c4b_fp16_96x197x64x197")):
            inp = S.config_inputs(name)
            t = timed(lambda: ref.gemm(inp["A"], inp["B"], adt=S.F16, bdt=S.F16))
            out[key] = {"value": C4_FLOP / t / 1e9, "unit": "GFLOP/s", "cores": 1,
                        "kind": "port", "sample": f"config {name} in full",
                        "seconds_full_config": t}
    if "ln" in only:
        inp = S.config_inputs("c5_ln")
        t = timed(lambda: ref.layer_norm(inp["x"], inp["gamma"], inp["beta"]))
        out["c5_layer_norm_f32_16384x4096"] = {
            "value": LN_BYTES / t / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": "config 5 LayerNorm in full", "seconds_full_config": t}
    if "sce" in only:
        inp = S.config_inputs("c5_sce")
        t = timed(lambda: ref.sce(inp["logits"], inp["labels"]))
        out["c5_sce_f32_4096x32000"] = {
            "value": SCE_BYTES / t / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": "config 5 SCE (mean loss) in full", "seconds_full_config": t}
    return out


class PowerSampler:
    """Samples `amd-smi metric -g 0 --power --clock --json` in a thread
    (each call takes ~0.1 s) while a workload runs: socket power and the
    mean of the graphics clocks of the eight XCDs."""

    def __init__(self):
        import threading
        self.samples, self._stop = [], threading.Event()
        self._th = threading.Thread(target=self._run, daemon=True)

    def _run(self):
        import subprocess
        while not self._stop.is_set():
            try:
                r = subprocess.run(["amd-smi", "metric", "-g", "0", "--power", "--clock",
                                    "--json"], capture_output=True, text=True, timeout=20)
                d = json.loads(r.stdout)
                g = d["gpu_data"][0] if isinstance(d, dict) else d[0]
                p = g["power"]["socket_power"]
                clks = [v["clk"]["value"] for k, v in g["clock"].items()
                        if k.startswith("gfx_") and isinstance(v, dict)
                        and isinstance(v.get("clk"), dict)]
                if isinstance(p, dict) and clks:
                    self.samples.append((float(p["value"]), sum(clks) / len(clks)))
            except Exception:  # a missing or failing amd-smi leaves no sample
                time.sleep(0.2)

    def __enter__(self):
        self._th.start()
        return self

    def __exit__(self, *exc):
        self._stop.set()
        self._th.join()

    def summary(self):
        if not self.samples:
            return {"samples": 0}
        pw = sorted(x[0] for x in self.samples)
        ck = sorted(x[1] for x in self.samples)
        return {"samples": len(pw), "power_w_median": pw[len(pw) // 2], "power_w_max": pw[-1],
                "gfx_clock_mhz_median": ck[len(ck) // 2]}


def telemetry(args, torch, nh, S):
    """Board power and graphics clock (amd-smi) while each workload runs
    back to back for args.telemetry_seconds: config 2 on this library's
    kernel, on hipBLASLt (torch.bmm), config 3 on this library's kernel, and
    a loop of nothing but bf16 MFMAs
    (nova-compiler_amd/libnova_probe.so, no memory traffic).  The MFMA busy
    fraction follows as TFLOP/s / (peak x clock / 2.4 GHz)."""
    import ctypes
    out = {}

    def drive(fn, flop):
        t0 = time.time()
        while time.time() - t0 < 1.0:          # settle the clock
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        n = 0
        with PowerSampler() as ps:
            e0.record()
            t0 = time.time()
            while time.time() - t0 < args.telemetry_seconds:
                for _ in range(20):
                    fn()
                n += 20
                torch.cuda.synchronize()
            e1.record()
            torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / n
        r = {"ms": ms, "tflops": flop / (ms * 1e-3) / 1e12, "calls": n}
        r.update(ps.summary())
        # One line per workload: the stage runs for minutes in all.
        print(f"[bench] telemetry: {r['tflops']:.1f} TFLOP/s, {r.get('samples', 0)} samples",
              file=sys.stderr, flush=True)
        if r.get("gfx_clock_mhz_median"):
            r["mfma_busy_at_clock"] = r["tflops"] / (PEAK_BF16_TFLOPS * r["gfx_clock_mhz_median"]
                                                     / 2400.0)
        return r

    inp = S.config_inputs("c2")
    A = to_dev(inp["A"], S.BF16, torch)
    B = to_dev(inp["B"], S.BF16, torch)
    del inp
    C = torch.empty(8, 4096, 4096, device="cuda", dtype=torch.float32)
    d = [nh.ref(nh.memref_of(t)) for t in (A, B, C)]
    f_ = nh.lib()._mlir_ciface_nova_hip_batch_matmul_bf16_f32
    nh._bind_stream()
    out["c2_gemm_pers_kernel"] = drive(lambda: f_(*d), C2_FLOP)
    out["c2_hipblaslt"] = drive(lambda: torch.bmm(A, B, out_dtype=torch.float32, out=C), C2_FLOP)
    # The same product with B stored K-contiguous (a transposed copy, passed
    # as a view): the kernel reads B's fragments with plain 16-byte LDS reads
    # instead of transposing ones; everything else is unchanged.
    Bt = B.transpose(1, 2).contiguous()
    dt = [nh.ref(nh.memref_of(t)) for t in (A, Bt.transpose(1, 2), C)]
    out["c2_gemm_pers_kernel_b_k_contiguous"] = drive(lambda: f_(*dt), C2_FLOP)
    del A, B, Bt, C
    torch.cuda.empty_cache()
    inp = S.config_inputs("c3")
    x = to_dev(inp["x"], S.BF16, torch)
    W = to_dev(inp["W"], S.BF16, torch)
    b = to_dev(inp["bias"], S.BF16, torch)
    del inp
    y = torch.empty(4096, 11008, device="cuda", dtype=torch.bfloat16)
    d3 = [nh.memref_of(t) for t in (x, W.t(), b, y)]
    r3 = [nh.ref(v) for v in d3]
    f3 = nh.lib()._mlir_ciface_nova_hip_linear_bf16_bias_gelu
    out["c3_gemm_pers_kernel"] = drive(lambda: f3(*r3), C3_FLOP)
    del x, W, b, y, d3, r3
    torch.cuda.empty_cache()
    probe = ctypes.CDLL(os.path.join(REPO, "nova-compiler_amd", "libnova_probe.so"))
    probe.nova_probe_mfma_loop.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                           ctypes.c_void_p, ctypes.POINTER(ctypes.c_double)]
    buf = torch.empty(256 * 256, device="cuda")
    flop = ctypes.c_double(0.0)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def mfma():
        rc = probe.nova_probe_mfma_loop(ctypes.c_void_p(buf.data_ptr()), 256, 20000, stream,
                                        ctypes.byref(flop))
        if rc:
            raise RuntimeError(f"probe launch failed: {rc}")

    mfma()
    torch.cuda.synchronize()
    out["mfma_only_probe"] = drive(mfma, flop.value)
    probe.nova_probe_mfma_loop16.argtypes = probe.nova_probe_mfma_loop.argtypes
    flop16 = ctypes.c_double(0.0)

    def mfma16():
        rc = probe.nova_probe_mfma_loop16(ctypes.c_void_p(buf.data_ptr()), 256, 20000, stream,
                                          ctypes.byref(flop16))
        if rc:
            raise RuntimeError(f"probe launch failed: {rc}")

    mfma16()
    torch.cuda.synchronize()
    out["mfma_only_probe_16x16x32"] = drive(mfma16, flop16.value)
    # The GEMM's per-K-step work from an L2-resident source, its operands
    # staged into LDS by LDS-DMA or by loads into registers plus ds_write.
    probe.nova_probe_stage.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                       ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                       ctypes.POINTER(ctypes.c_double)]
    probe.nova_probe_stage_src_bytes.restype = ctypes.c_int64
    nsrc = probe.nova_probe_stage_src_bytes() // 2
    src = torch.randn(nsrc, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16).cuda()
    for name, dma in (("lds_dma", 1), ("registers_ds_write", 0), ("lds_dma_transposing_b", 2)):
        fl = ctypes.c_double(0.0)

        def staged(dma=dma, fl=fl):
            rc = probe.nova_probe_stage(ctypes.c_void_p(src.data_ptr()),
                                        ctypes.c_void_p(buf.data_ptr()), 256, 2000, dma,
                                        stream, ctypes.byref(fl))
            if rc:
                raise RuntimeError(f"probe launch failed: {rc}")

        staged()
        torch.cuda.synchronize()
        out[f"staging_probe_{name}"] = drive(staged, fl.value)
    out["note"] = ("amd-smi socket power and mean XCD graphics clock, medians over the samples; "
                   "mfma_busy_at_clock = TFLOP/s / (2516.6 x clock / 2400 MHz)")
    return out


def cpu_model():
    """The host CPU's model name, from /proc/cpuinfo."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only; --gpus {args.gpus} is not "
              "supported (the multi-GPU sharding plan is design-only).", file=sys.stderr)
        sys.exit(2)
    import torch
    import nova_hip as nh
    import nova_seed as S
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    torch.cuda.set_device(0)
    nh.lib()
    only = (set(args.only.split(",")) if args.only else
            {"c1", "c2", "c3", "c4", "ln", "sce", "sce_bwd", "sce_fwd_bwd", "ln_bwd", "c3_bwd",
             "c2_vendor", "gpt_step"})
    cfg = {}

    def stage(name, f):
        t0 = time.time()
        print(f"[bench] {name} ...", file=sys.stderr, flush=True)
        _LAUNCH_STATS.clear()
        r = f()
        if isinstance(r, dict) and _LAUNCH_STATS:
            r["launch_ms"] = dict(_LAUNCH_STATS)
        print(f"[bench] {name}: {json.dumps(r)} ({time.time() - t0:.1f} s)", file=sys.stderr,
              flush=True)
        torch.cuda.empty_cache()
        return r

    c2 = stage("c2", lambda: bench_c2(args, torch, nh, S)) if "c2" in only else None
    if "c1" in only:
        cfg["c1_matmul_f32_256"] = stage("c1", lambda: bench_c1(args, torch, nh, S))
    if "c3" in only:
        cfg["c3_linear_bias_gelu_bf16"] = stage("c3", lambda: bench_c3(args, torch, nh, S))
    if "c4" in only:
        cfg["c4a_fp16_96x197x197x64"] = stage("c4a", lambda: bench_c4(args, torch, nh, S, "c4a", C4A_BYTES))
        cfg["c4b_fp16_96x197x64x197"] = stage("c4b", lambda: bench_c4(args, torch, nh, S, "c4b", C4B_BYTES))
    if "ln" in only:
        cfg["c5_layer_norm_f32_16384x4096"] = stage("ln", lambda: bench_ln(args, torch, nh, S))
    if "sce" in only:
        cfg["c5_sce_f32_4096x32000"] = stage("sce", lambda: bench_sce(args, torch, nh, S))
    if "sce_bwd" in only:
        cfg["c5_sce_backward_f32_4096x32000"] = stage(
            "sce_bwd", lambda: bench_sce_bwd(args, torch, nh, S, False))
    if "sce_fwd_bwd" in only:
        cfg["c5_sce_fwd_bwd_f32_4096x32000"] = stage(
            "sce_fwd_bwd", lambda: bench_sce_bwd(args, torch, nh, S, True))
    if "ln_bwd" in only:
        cfg["c5_layer_norm_backward_f32_16384x4096"] = stage(
            "ln_bwd", lambda: bench_ln_bwd(args, torch, nh, S))
    if "c3_bwd" in only:
        cfg["c3_linear_backward_bf16_f32"] = stage("c3_bwd", lambda: bench_c3_bwd(args, torch, nh, S))
    if "gpt_step" in only:
        cfg["gpt_step_f32_nova_run_8x1024_v50304"] = stage("gpt_step", lambda: bench_gpt_step(args, torch))
    if "c2_vendor" in only:
        cfg["c2_vendor_hipblaslt_reference"] = stage("c2_vendor", lambda: bench_c2_vendor(args, torch, S))
    if "copy" in only:  # calibration only; not part of the default run
        cfg["hbm_copy_256MiB"] = stage("copy", lambda: bench_copy(args, torch))
    if only & {"ln", "sce", "sce_bwd", "sce_fwd_bwd", "ln_bwd", "copy"}:
        ceil = stage("copy_ceiling", lambda: bench_copy_ceiling(args, torch))
        cfg["hbm_copy_ceiling_256MiB"] = ceil
        for key, r in cfg.items():
            if key.startswith("c5_") and isinstance(r, dict) and "gbs" in r and "gbs" in ceil:
                r["frac_copy_ceiling"] = r["gbs"] / ceil["gbs"]

    tele = stage("telemetry", lambda: telemetry(args, torch, nh, S)) if args.telemetry else None

    cpu = None
    if not args.no_cpu_baseline:
        cpu = stage("cpu_baseline", lambda: cpu_baseline(S))
        # The oracle on one core for each other config of BASELINE.json, in
        # full where that takes seconds, config 3 on a slab (extrapolated),
        # reported beside the config it belongs to.
        per = stage("cpu_baselines", lambda: cpu_baselines(S, only))
        for key, c in per.items():
            if key in cfg and isinstance(cfg[key], dict):
                cfg[key]["cpu_baseline"] = c
                if "ms" in cfg[key] and c.get("seconds_full_config"):
                    cfg[key]["gpu_over_cpu"] = c["seconds_full_config"] / (cfg[key]["ms"] * 1e-3)
            else:
                cfg[key] = {"cpu_baseline": c}

    # HBM bytes per config-2 launch: two rocprofv3 --pmc runs (FETCH_SIZE,
    # WRITE_SIZE) of `bench.py --only c2`, scaled by the copy calibration and
    # committed under profiles/; counters cannot be read inside this run.
    traffic, traffic_src = None, None
    tpath = os.path.join(REPO, "profiles", "gemm_c2_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")
        traffic_src = ("profiles/gemm_c2_traffic.json (committed rocprofv3 FETCH_SIZE + "
                       "WRITE_SIZE measurement of bench.py --only c2, calibrated on a copy; "
                       "not measured in this run)")

    head = c2 or {"ms": float("nan"), "tflops": float("nan"), "frac_mfma": float("nan")}
    line = {
        "metric": "batch-GEMM TFLOP/s & % MFMA peak; reduction HBM GB/s & % peak (1 MI355X)",
        "value": head["tflops"],
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms"],
        # Single-launch times of config 2 (a second pass, events between launches).
        "launch_ms": head.get("launch_ms"),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded counter-based generator (nova-compiler_amd/host/nova_seed.c), "
                "A,B uniform[-1,1] seed 1",
        "config": {"workload": "c2: linalg.batch_matmul bf16 x bf16 -> f32 accumulate/output, "
                               "batch=8, M=N=K=4096",
                   "kernel": "gemm_pers_kernel: persistent, one workgroup per CU, 256x256x64 tiles, 2-stage LDS-DMA ring, v_mfma_f32_32x32x16_bf16",
                   "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": head["tflops"], "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": head["frac_mfma"], "traffic": traffic,
                     "traffic_source": traffic_src},
        "cpu_baseline": cpu,
        "configs": cfg,
    }
    if tele is not None:
        line["telemetry"] = tele
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
