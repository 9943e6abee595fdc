"""Benchmark of the TCFP-12 hot path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--part all|gemm|quant|block|mlp|c5|copy|scaled_mm]

Headline (BASELINE.json ``metric``, configs[1]): the fused dual-FP8 GEMM
``out = X W_hi^T s_x s_hi + X W_lo^T s_x s_lo`` at M = N = K = 4096,
per-tensor scales, FP32 accumulation, bf16 output, inputs resident in HBM.
One step = one dual-GEMM launch; ``value`` is TFLOP/s counting the dual as
two GEMMs (2 * 2 * 4096^3 FLOP per step).

The same JSON line carries the roofline of that kernel (HIP events on the
stream the kernel runs on), the CPU baseline (the reference's CPU path --
quantisation and fp32 matmuls of the dequantised operands -- on the same
problem, on the box's host cores), and secondary figures:
library comparators at the same shape, the dual-quant kernels' HBM rate,
and the 1024 -> 4096 -> 1024 MLP training step against BF16.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

FP8_PEAK_TFLOPS = 5000.0   # MI355X dense FP8 MFMA (AMD published)
BF16_PEAK_TFLOPS = 2500.0  # MI355X dense BF16 MFMA
HBM_PEAK_GBS = 8000.0      # MI355X HBM3E


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def event_time_ms(fn, iters, stream, warmup=3):
    """Average time per call of ``fn`` over ``iters`` calls, from HIP events
    on ``stream`` (the stream the kernels are launched on), after
    ``warmup`` untimed calls (the first launch of a kernel also loads its
    code object)."""
    import torch

    for _ in range(warmup):
        fn()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(iters):
        fn()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / iters


def c2_tensors():
    """configs[1] operands resident in HBM: X = seeded bf16 N(0,1) quantised
    per tensor, W = seeded fp32 N(0,1) dual-quantised (no EF)."""
    import torch

    from tcfp_amd import kernels as K

    dev = torch.device("cuda:0")
    n = 4096
    xb = torch.randn(n, n, generator=torch.Generator().manual_seed(0)).bfloat16().to(dev)
    w = torch.randn(n, n, generator=torch.Generator().manual_seed(1)).to(dev)
    a, sa = K.quantize_per_tensor(xb)
    h, l, ih, il = K.dual_quantize_per_tensor(w)
    torch.cuda.synchronize()
    return (a, h, l, sa, ih, il, xb, w)


def bench_dual_gemm(steps, warmup, t=None, sustained=0):
    """The headline: ``warmup`` untimed launches, then exactly ``steps``
    launches timed by wall clock (synchronised on both sides) and by HIP
    events on the launch stream.

    ``sustained`` > 0 first measures the same kernel back to back over that
    many launches (HIP events; reported beside the headline).  From an idle
    GPU -- even 50 ms idle -- the first ~200 launches run 120-143 us while
    the board's power management ramps up, against 106-110 us back to back
    (measured per 20 launches); the sustained run puts the headline's
    timed steps in the working state a training loop keeps the GPU in."""
    import torch

    from tcfp_amd import kernels as K

    dev = torch.device("cuda:0")
    if t is None:
        t = c2_tensors()
    a, h, l, sa, ih, il, xb, w = t
    n = a.shape[0]
    out = torch.empty(n, n, dtype=torch.bfloat16, device=dev)

    def step():
        return K.fused_dual_gemm_forward(a, h, l, sa, ih, il, out_dtype=torch.bfloat16)

    stream = torch.cuda.current_stream(dev)
    res = {}
    if sustained:
        ms = event_time_ms(step, sustained, stream, warmup=1)
        res["sustained_launches"] = sustained
        res["sustained_ms"] = ms
        res["sustained_tflops"] = 2 * 2 * n**3 / (ms * 1e-3) / 1e12
    for _ in range(warmup):
        out = step()
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(steps):
        out = step()
    ev1.record(stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    wall_ms = (t1 - t0) * 1e3 / steps
    kern_ms = ev0.elapsed_time(ev1) / steps
    flop = 2 * 2 * n**3
    res.update({
        "n": n, "flop": flop, "wall_ms": wall_ms, "kern_ms": kern_ms,
        "tflops_wall": flop / (wall_ms * 1e-3) / 1e12,
        "tflops_kern": flop / (kern_ms * 1e-3) / 1e12,
    })
    # parity of the timed output against a torch fp32 dequant matmul
    ref = (a.float() * sa) @ (h.float() * ih + l.float() * il).t()
    res["rel_fro"] = ((out.float() - ref).norm() / ref.norm()).item()
    res["tensors"] = t
    return res


def bench_scaled_mm(steps, warmup):
    """hipBLASLt's single ``torch._scaled_mm`` on C2's operands (the
    comparator arm of ``bench_comparators``) alone: ``warmup`` untimed calls,
    then ``steps`` timed by HIP events -- a workload for counter runs."""
    import torch

    a, h, l, sa, ih, il, xb, w = c2_tensors()
    ms = event_time_ms(lambda: torch._scaled_mm(a, h.t(), scale_a=sa, scale_b=ih,
                                                out_dtype=torch.bfloat16),
                       steps, torch.cuda.current_stream(), warmup=warmup)
    return {"scaled_mm_single_ms": ms, "tflops": 2 * a.shape[0] ** 3 / ms / 1e9}


def bench_comparators(t, iters=200, heat=300, rounds=3):
    """Library comparators at C2's shape, each measured in the same working
    state as the dual GEMM: per round, ``heat`` untimed back-to-back calls
    (the power ramp from idle lasts ~200 launches), then ``iters`` calls
    timed by HIP events; the median over ``rounds`` interleaved rounds.
    Arms: this build's dual GEMM on C2's data, hipBLASLt's single
    ``torch._scaled_mm``, the reference's naive tier (2 x ``_scaled_mm`` +
    add), BF16 ``torch.matmul``, and -- a diagnostic of the power limit, not
    a result -- the dual GEMM on all-zero operands (no bit toggles in the
    MFMA datapath)."""
    import torch

    from tcfp_amd import kernels as K

    a, h, l, sa, ih, il, xb, w = t
    stream = torch.cuda.current_stream()
    n = a.shape[0]
    wb = w.bfloat16()
    az, hz, lz = torch.zeros_like(a), torch.zeros_like(h), torch.zeros_like(l)
    arms = {
        "dual_c2_data": (4, lambda: K.fused_dual_gemm_forward(a, h, l, sa, ih, il,
                                                              out_dtype=torch.bfloat16)),
        "scaled_mm_single": (2, lambda: torch._scaled_mm(a, h.t(), scale_a=sa, scale_b=ih,
                                                         out_dtype=torch.bfloat16)),
        "naive_2x_scaled_mm_add": (4, lambda: torch._scaled_mm(
            a, h.t(), scale_a=sa, scale_b=ih, out_dtype=torch.bfloat16) + torch._scaled_mm(
            a, l.t(), scale_a=sa, scale_b=il, out_dtype=torch.bfloat16)),
        "bf16_matmul": (2, lambda: xb @ wb.t()),
        "dual_zero_operands": (4, lambda: K.fused_dual_gemm_forward(
            az, hz, lz, sa, ih, il, out_dtype=torch.bfloat16)),
    }
    res = {}
    times = {k: [] for k in arms}
    for _ in range(rounds):
        for k, (_, fn) in list(arms.items()):
            try:
                times[k].append(event_time_ms(fn, iters, stream, warmup=heat))
            except Exception as e:  # library path unavailable on this build
                res[f"{k}_error"] = str(e)[:200]
                arms.pop(k)
    for k, (mult, _) in arms.items():
        ms = statistics.median(times[k])
        res[f"{k}_ms"] = ms
        res[f"{k}_tflops"] = mult * n**3 / (ms * 1e-3) / 1e12
    res["method"] = (f"per arm and round: {heat} untimed calls then {iters} timed (HIP events); "
                     f"median of {rounds} interleaved rounds")
    return res


def bench_block_gemms(iters=100, heat=300, rounds=3):
    """block-scaled dual GEMM at 4096^3, bs 32/64/128 (int8
    power-of-two exponents, the reference's block format, and fp32
    448/amax block scales, the configuration's literal form), plus the
    single block-scaled GEMM at bs 64.  fp32 out, as the reference's
    kernels.  Timed as the comparators are: per arm and round, ``heat``
    untimed back-to-back calls (out of the idle clock state), then
    ``iters`` calls timed by HIP events; the median of ``rounds``
    interleaved rounds.  (``--part block`` keeps the short form, 3 untimed
    and 20 timed calls per arm, for the profiler runs.)"""
    import torch

    from tcfp_amd import kernels as K

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    n = 4096
    x = torch.randn(n, n, generator=torch.Generator().manual_seed(0)).bfloat16().to(dev)
    w = torch.randn(n, n, generator=torch.Generator().manual_seed(1)).to(dev)
    arms = {}  # name -> (GEMMs per call, fn)
    for bs in (32, 64, 128):
        a, ea = K.block_quantize_fp8(x, bs)
        h, l, eh, el = K.fused_dual_quantize_fp8(w, bs)
        arms[f"block{bs}_dual"] = (
            2, lambda a=a, h=h, l=l, ea=ea, eh=eh, el=el, bs=bs:
            K.fused_block_scaled_dual_gemm_forward(a, h, l, ea, eh, el, bs))
        if bs == 64:
            arms["block64_single"] = (
                1, lambda a=a, h=h, ea=ea, eh=eh: K.block_scaled_gemm(a, h, ea, eh, 64))
        a, sa = K.block_quantize_fp8(x, bs, scale_format="fp32")
        h, l, sh, sl = K.fused_dual_quantize_fp8(w, bs, scale_format="fp32")
        arms[f"block{bs}_f32s_dual"] = (
            2, lambda a=a, h=h, l=l, sa=sa, sh=sh, sl=sl, bs=bs:
            K.fused_block_scaled_dual_gemm_forward(a, h, l, sa, sh, sl, bs))
    times = {k: [] for k in arms}
    for _ in range(rounds):
        for k, (_, fn) in arms.items():
            times[k].append(event_time_ms(fn, iters, stream, warmup=heat))
    res = {}
    for k, (mult, _) in arms.items():
        ms = statistics.median(times[k])
        res[f"{k}_ms"] = ms
        res[f"{k}_tflops"] = 2 * mult * n**3 / (ms * 1e-3) / 1e12
    res["method"] = (f"per arm and round: {heat} untimed calls then {iters} timed (HIP events); "
                     f"median of {rounds} interleaved rounds")
    return res


def bench_copy(steps):
    """Calibration workload for the PMC traffic counters: a plain device
    copy of 256 MiB (256 MiB read + 256 MiB written per launch)."""
    import torch

    dev = torch.device("cuda:0")
    src = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    return {"copy_bytes_each_way": 256 << 20, "launches": steps}


def rotated_time_ms(calls, rounds, stream):
    """Average time per call over ``rounds`` passes of ``calls`` (one call
    per independent set of inputs and outputs), HIP events on ``stream``:
    with the sets together well beyond the 256 MB Infinity Cache every call
    reads its operands from HBM (the cold figure).  One untimed pass
    first."""
    import torch

    for fn in calls:
        fn()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(rounds):
        for fn in calls:
            fn()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / (rounds * len(calls))


COLD_BYTES = 768 << 20  # working set of the cold protocol: 3 x the Infinity Cache


def bench_gemm_sweep(iters=50, rounds=3):
    """Per-tensor dual FP8 GEMM over the configs' shapes and a K sweep
    (M x N x K, fp32 and bf16 output, E4M3 operands, no bias), plus the
    single FP8 GEMM at the wgrad shapes: median of ``rounds`` event-timed
    runs of ``iters`` back-to-back launches each.  The K sweep separates
    the main loop's rate (the slope) from a GEMM's fixed cost (the
    intercept: prologue and the output written)."""
    import torch

    from tcfp_amd import kernels as K

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    out = {}

    def timed(fn):
        return sorted(event_time_ms(fn, iters, stream) for _ in range(rounds))[rounds // 2]

    shapes = [(8192, 4096, k) for k in (1024, 2048, 4096, 8192)] + \
             [(8192, 1024, k) for k in (1024, 2048, 4096, 8192)] + [(4096, 4096, 4096)]
    # out of the idle-to-busy clock ramp first (1500 back-to-back launches)
    g = torch.Generator(device=dev).manual_seed(1)
    a, sa = K.quantize_per_tensor(torch.randn(4096, 4096, device=dev, generator=g))
    h, l, ih, il = K.dual_quantize_per_tensor(torch.randn(4096, 4096, device=dev, generator=g))
    for _ in range(1500):
        K.fused_dual_gemm_forward(a, h, l, sa, ih, il, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    for (m, n, k) in shapes:
        g = torch.Generator(device=dev).manual_seed(m + n + k)
        a, sa = K.quantize_per_tensor(torch.randn(m, k, device=dev, generator=g))
        h, l, ih, il = K.dual_quantize_per_tensor(torch.randn(n, k, device=dev, generator=g))
        for od in (torch.float32, torch.bfloat16):
            ms = timed(lambda: K.fused_dual_gemm_forward(a, h, l, sa, ih, il, out_dtype=od))
            key = f"dual_{m}x{n}x{k}_{'f32' if od == torch.float32 else 'bf16'}"
            out[key] = {"ms": ms, "tflops": 4.0 * m * n * k / (ms * 1e-3) / 1e12}
    for (m, n, k) in ((4096, 1024, 8192), (1024, 4096, 8192)):
        g = torch.Generator(device=dev).manual_seed(m + n + k)
        a, sa = K.quantize_per_tensor(torch.randn(m, k, device=dev, generator=g),
                                      torch.float8_e5m2)
        b, sb = K.quantize_per_tensor(torch.randn(n, k, device=dev, generator=g))
        ms = timed(lambda: K.fp8_gemm_nt(a, b, sa, sb))
        out[f"single_{m}x{n}x{k}_f32"] = {"ms": ms, "tflops": 2.0 * m * n * k / (ms * 1e-3) / 1e12}
    return out


def bench_quant_in_consumer(iters=50, rounds=5):
    """Quantisation inside the consuming GEMM against a separate pass, at
    the C4 gradient's consumer shapes: this build's in-GEMM activation
    quantisation (the block-scaled act-quant GEMM, a11) against
    ``block_quantize_fp8`` + the block dual GEMM on the same operands (the
    results are identical; the in-GEMM form re-quantises each activation
    panel once per output-column tile).  Median of ``rounds``."""
    import torch

    from tcfp_amd import kernels as K

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    bs = 64
    out = {}
    for (m, n, k) in ((8192, 4096, 1024), (8192, 1024, 4096), (8192, 512, 1024)):
        g = torch.Generator(device=dev).manual_seed(1)
        x = torch.randn(m, k, device=dev, generator=g)
        w = torch.randn(n, k, device=dev, generator=g) * 0.02
        h, l, eh, el = K.fused_dual_quantize_fp8(w, bs)

        def fused():
            return K.fused_act_quant_dual_gemm_forward(x, h, l, eh, el, bs,
                                                       save_side_outputs=False)[0]

        def sep():
            aq, ea = K.block_quantize_fp8(x, bs)
            return K.fused_block_scaled_dual_gemm_forward(aq, h, l, ea, eh, el, bs)

        same = bool(torch.equal(fused(), sep()))
        tf = sorted(event_time_ms(fused, iters, stream) for _ in range(rounds))[rounds // 2]
        ts = sorted(event_time_ms(sep, iters, stream) for _ in range(rounds))[rounds // 2]
        out[f"{m}x{n}x{k}_fp32"] = {"in_gemm_ms": tf, "separate_ms": ts, "identical": same}
    return out


def bench_dual_quant_cold(rounds=10):
    """Only the cold rotation of the per-tensor dual-quant + EF row at
    4096^2 (five W + EF sets, 640 MB), for profiling its kernels and
    traffic under the cold protocol."""
    import torch

    from tcfp_amd import kernels as K

    dev = torch.device("cuda:0")
    sets = []
    for i in range(5):
        g = torch.Generator(device=dev).manual_seed(100 + i)
        sets.append((torch.randn(4096, 4096, device=dev, generator=g) * 0.02,
                     torch.zeros(4096, 4096, device=dev)))
    calls = [lambda w=w, ef=ef: K.dual_quantize_per_tensor(w, ef) for w, ef in sets]
    ms = rotated_time_ms(calls, rounds, torch.cuda.current_stream(dev))
    return {"per_tensor_ef_4096x4096_cold_ms": ms,
            "per_tensor_ef_4096x4096_cold_GBs": 14 * 4096 * 4096 / (ms * 1e-3) / 1e9,
            "calls": rounds * len(calls) + len(calls)}


def bench_dual_quant(iters=20, cold_rounds=4):
    """The quantisation kernels at the sizes the configs use, each timed two
    ways: warm (``iters`` back-to-back calls on one set of buffers, which
    can stay in the 256 MB Infinity Cache) and cold (calls rotating over
    independent buffer sets totalling >= 768 MB, ``rotated_time_ms``).
    GB/s = algorithmic bytes (each input read once, each output written
    once) / time."""
    import torch

    from tcfp_amd import kernels as K
    from tcfp_amd.core import ErrorFeedbackState

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    out = {}

    def row(name, make, alg_bytes, set_bytes):
        """make(i) -> a zero-argument call on buffer set i."""
        f0 = make(0)
        ms = event_time_ms(f0, iters, stream)
        nsets = max(2, -(-COLD_BYTES // set_bytes))
        calls = [f0] + [make(i) for i in range(1, nsets)]
        cold = rotated_time_ms(calls, cold_rounds, stream)
        out[f"{name}_ms"] = ms
        out[f"{name}_GBs"] = alg_bytes / (ms * 1e-3) / 1e9
        out[f"{name}_cold_ms"] = cold
        out[f"{name}_cold_GBs"] = alg_bytes / (cold * 1e-3) / 1e9
        out[f"{name}_cold_sets"] = nsets
        del calls
        torch.cuda.empty_cache()

    n, k = 4096, 4096
    ne = n * k

    def wef(i, rows=n):
        g = torch.Generator(device=dev).manual_seed(100 + i)
        return (torch.randn(rows, k, device=dev, generator=g) * 0.02,
                torch.zeros(rows, k, device=dev))

    # per-tensor with EF (update in place): 14 algorithmic B/elem (W and EF
    # read, EF written, two code arrays); a set holds W, EF and the codes
    def per_tensor(i):
        w, ef = wef(i)
        return lambda: K.dual_quantize_per_tensor(w, ef)

    row("per_tensor_ef_4096x4096", per_tensor, 14 * ne, 10 * ne)

    # the same with delayed scaling on a non-validation step (the residual
    # amax is predicted: two passes over W + EF instead of three)
    def delayed(i):
        w, ef = wef(i)
        st = ErrorFeedbackState(residual_validation_interval=10**9)
        K.dual_quantize_per_tensor_delayed(w, ef, st, "w")  # the first call validates
        return lambda: K.dual_quantize_per_tensor_delayed(w, ef, st, "w")

    row("per_tensor_ef_delayed_4096x4096", delayed, 14 * ne, 10 * ne)

    # NF-aware W_hi scaling (sigma = 3): the first pass also sums v and v^2
    def nf(i):
        w, ef = wef(i)
        return lambda: K.dual_quantize_per_tensor(w, ef, sigma_factor=3.0)

    row("per_tensor_ef_nf_4096x4096", nf, 14 * ne, 10 * ne)

    # block-64 with EF: 14 + 2/64 B/elem
    def block64(i):
        w, ef = wef(i)
        return lambda: K.fused_dual_quantize_fp8(w, 64, error_buf=ef)

    row("block64_ef_4096x4096", block64, (14 + 2 / 64) * ne, 10 * ne)

    # SRR block-64 on the C5 scale-up weight [16384, 4096]: 6 + 2/64 B/elem
    def srr(i):
        g = torch.Generator(device=dev).manual_seed(200 + i)
        w2 = torch.randn(16384, 4096, device=dev, generator=g) * 0.02
        return lambda: K.fused_dual_quantize_fp8(w2, 64, stochastic_lo=True, seed=1)

    row("block64_srr_16384x4096", srr, (6 + 2 / 64) * 16384 * 4096, 6 * 16384 * 4096)

    # act quant bf16 [8192, 1024] -> e4m3: 2 + 1 B/elem
    def act(i):
        g = torch.Generator(device=dev).manual_seed(300 + i)
        x = torch.randn(8192, 1024, device=dev, generator=g).bfloat16()
        return lambda: K.quantize_per_tensor(x)

    row("act_quant_bf16_8192x1024", act, 3 * 8192 * 1024, 3 * 8192 * 1024)
    return out


def bench_mlp(steps=100, time_iters=20, arms=("tcfp", "tcfp_fused", "bf16", "fp32"), rounds=5):
    """1024 -> 4096 -> 1024 GELU MLP, 8192 tokens, MSE, AdamW 1e-3.

    Arms: TCFP-12 (both linears converted, per-tensor scales with EF: the
    drop-in TCFPLinear path), the same with the GELU fused into the
    quantisation around it (``fuse_tcfp_mlp``; bit-identical results),
    BF16 autocast (the target's baseline), and the same model in fp32 (the
    reference harness's "BF16" baseline is an fp32 model,
    benchmarks/benchmark_tcfp.py:482-516; context only).  Each arm trains
    ``steps`` steps (the losses); then the arms are timed in ``rounds``
    interleaved rounds of ``time_iters`` steps each (HIP events), and each
    arm's median round is reported, so that clock drift over the run falls
    on every arm alike."""
    import torch
    import torch.nn as nn

    from tcfp_amd.nn import convert_to_tcfp, fuse_tcfp_mlp

    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(0)
    x = torch.randn(8192, 1024, generator=g).bfloat16().to(dev)
    y = torch.randn(8192, 1024, generator=g).to(dev)

    def make(arm):
        torch.manual_seed(1)
        m = nn.Sequential(nn.Linear(1024, 4096), nn.GELU(), nn.Linear(4096, 1024)).to(dev)
        if arm.startswith("tcfp"):
            convert_to_tcfp(m, use_tensor_cores=True)
        if arm == "tcfp_fused":
            m = fuse_tcfp_mlp(m)
        return m

    xf = x.float()

    def train(arm):
        m = make(arm)
        opt = torch.optim.AdamW(m.parameters(), lr=1e-3)

        def step():
            if arm.startswith("tcfp"):
                out = m(x)
            elif arm == "fp32":
                out = m(xf)
            else:
                with torch.autocast("cuda", dtype=torch.bfloat16):
                    out = m(x)
            loss = (out.float() - y).square().mean()
            opt.zero_grad(set_to_none=True)
            loss.backward()
            opt.step()
            return loss

        losses = []
        for i in range(steps):
            losses.append(step())
        torch.cuda.synchronize()
        return [float(v) for v in torch.stack(losses).detach().cpu()], step

    trained = {arm: train(arm) for arm in arms}
    stream = torch.cuda.current_stream(dev)
    times = {arm: [] for arm in arms}
    for _ in range(rounds):
        for arm in arms:
            times[arm].append(event_time_ms(trained[arm][1], time_iters, stream))
    ms_of = {arm: sorted(v)[len(v) // 2] for arm, v in times.items()}

    def run(arm):
        return trained[arm][0], ms_of[arm]

    res = {"steps": steps}
    if "tcfp" in arms:
        l_t, ms_t = run("tcfp")
        res.update({"tcfp_step_ms": ms_t, "loss_step1_tcfp": l_t[0],
                    f"loss_step{steps}_tcfp": l_t[-1]})
    if "bf16" in arms:
        l_b, ms_b = run("bf16")
        res.update({"bf16_autocast_step_ms": ms_b, f"loss_step{steps}_bf16": l_b[-1]})
    if "tcfp_fused" in arms:
        l_u, ms_u = run("tcfp_fused")
        res.update({"tcfp_fused_step_ms": ms_u, f"loss_step{steps}_tcfp_fused": l_u[-1]})
        if "tcfp" in arms:
            res["fused_losses_identical"] = l_u == l_t
    if "tcfp" in arms and "bf16" in arms:
        res["speedup_vs_bf16"] = ms_b / ms_t
        res[f"loss_rel_diff_step{steps}"] = abs(l_t[-1] - l_b[-1]) / l_b[-1]
    if "tcfp_fused" in arms and "bf16" in arms:
        res["speedup_fused_vs_bf16"] = ms_b / ms_u
    if "fp32" in arms:
        l_f, ms_f = run("fp32")
        res.update({"fp32_step_ms": ms_f, f"loss_step{steps}_fp32": l_f[-1]})
        if "tcfp" in arms:
            res["speedup_vs_fp32"] = ms_f / ms_t
    return res


def _tiny_gpt(vocab=256, d=256, layers=4, heads=4, ffn=1024, seq=128):
    """configs[4] model: decoder-only transformer (pre-LN, GELU FFN, tied
    head), the architecture of the reference's TinyGPT
    (examples/train_convergence.py:192-260) at BASELINE's vocab of 256.
    Attention runs in float32 with contiguous operands in both arms."""
    import torch
    import torch.nn as nn
    import torch.nn.functional as F

    class Attn(nn.Module):
        def __init__(self):
            super().__init__()
            self.h, self.dh = heads, d // heads
            self.qkv = nn.Linear(d, 3 * d)
            self.proj = nn.Linear(d, d)

        def forward(self, x):
            B, T, C = x.shape
            qkv = self.qkv(x).float().reshape(B, T, 3, self.h, self.dh)
            q, k, v = (t.transpose(1, 2).contiguous() for t in qkv.unbind(2))
            with torch.autocast("cuda", enabled=False):
                att = torch.matmul(q, k.transpose(-2, -1).contiguous()) / self.dh**0.5
                mask = torch.triu(torch.ones(T, T, device=x.device, dtype=torch.bool), 1)
                att = F.softmax(att.masked_fill(mask, float("-inf")), dim=-1)
                y = torch.matmul(att, v).transpose(1, 2).reshape(B, T, C).contiguous()
            return self.proj(y)

    class Block(nn.Module):
        def __init__(self):
            super().__init__()
            self.ln1, self.ln2 = nn.LayerNorm(d), nn.LayerNorm(d)
            self.attn = Attn()
            self.ffn = nn.Sequential(nn.Linear(d, ffn), nn.GELU(), nn.Linear(ffn, d))

        def forward(self, x):
            x = x + self.attn(self.ln1(x))
            return x + self.ffn(self.ln2(x))

    class TinyGPT(nn.Module):
        def __init__(self):
            super().__init__()
            self.tok = nn.Embedding(vocab, d)
            self.pos = nn.Embedding(seq, d)
            self.blocks = nn.ModuleList([Block() for _ in range(layers)])
            self.ln_f = nn.LayerNorm(d)
            self.head = nn.Linear(d, vocab, bias=False)
            self.head.weight = self.tok.weight
            for m in self.modules():
                if isinstance(m, nn.Linear):
                    nn.init.normal_(m.weight, std=0.02)
                    if m.bias is not None:
                        nn.init.zeros_(m.bias)
                elif isinstance(m, nn.Embedding):
                    nn.init.normal_(m.weight, std=0.02)

        def forward(self, idx):
            T = idx.shape[1]
            x = self.tok(idx) + self.pos(torch.arange(T, device=idx.device))
            for b in self.blocks:
                x = b(x)
            return self.head(self.ln_f(x).float())

    return TinyGPT()


def bench_c5(steps=50, time_iters=10, rounds=5):
    """TinyGPT (d 256, 4 layers, 4 heads, FFN 1024, vocab 256,
    seq 128, batch 32) with every QKV/O/FFN linear TCFP-12 block-64 + SRR,
    against BF16 autocast; and the 4096 -> 16384 -> 4096 scale-up layer at
    8192 tokens (peak memory and fwd+bwd time: block-64 SRR, block-64 EF,
    BF16).  The TinyGPT arms train ``steps`` steps each (the losses), then
    are timed in ``rounds`` interleaved rounds of ``time_iters`` steps
    (median): the step is host-bound, so it follows the host's state."""
    import torch
    import torch.nn as nn
    import torch.nn.functional as F

    from tcfp_amd.nn import convert_to_tcfp

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    g = torch.Generator().manual_seed(0)
    data = torch.randint(0, 256, (steps + rounds * (time_iters + 3) + 3, 32, 129),
                         generator=g).to(dev)
    res = {}
    step_of = {}
    for arm in ("tcfp_block64_srr", "bf16"):
        torch.manual_seed(1)
        model = _tiny_gpt().to(dev)
        if arm != "bf16":
            convert_to_tcfp(model, use_tensor_cores=True, scale_block_size=64, srr=True,
                            skip_patterns=("head",))
        opt = torch.optim.AdamW(model.parameters(), lr=3e-4, weight_decay=0.01)
        it = iter(range(data.shape[0]))

        def step(arm=arm, model=model, opt=opt, it=it):
            b = data[next(it)]
            with torch.autocast("cuda", dtype=torch.bfloat16, enabled=(arm == "bf16")):
                logits = model(b[:, :-1])
            loss = F.cross_entropy(logits.float().reshape(-1, 256), b[:, 1:].reshape(-1))
            opt.zero_grad(set_to_none=True)
            loss.backward()
            opt.step()
            return loss

        losses = [step() for _ in range(steps)]
        lv = [float(v) for v in torch.stack(losses).detach().cpu()]
        res[arm] = {"loss_first": lv[0], "loss_last": lv[-1], "steps": steps}
        step_of[arm] = step
    times = {arm: [] for arm in step_of}
    for _ in range(rounds):
        for arm, step in step_of.items():
            times[arm].append(event_time_ms(step, time_iters, stream, warmup=3))
    for arm in step_of:
        res[arm]["step_ms"] = statistics.median(times[arm])
    # (the TinyGPT arms are released before the scale-up layer's memory figures)
    step_of.clear()
    del step, model, opt, it
    res["loss_rel_diff_last"] = (abs(res["tcfp_block64_srr"]["loss_last"] - res["bf16"]["loss_last"])
                                 / res["bf16"]["loss_last"])
    # scale-up layer
    x = torch.randn(8192, 4096, generator=g).bfloat16().to(dev)
    from tcfp_amd.nn import set_block_dgrad, set_block_wgrad

    # the same layer with the opt-in FP8 block dgrad and / or the opt-in
    # single-pass bf16 wgrad
    for arm, kw in (("block64_srr", dict(scale_block_size=64, srr=True)),
                    ("block64_srr_fp8_dgrad", dict(scale_block_size=64, srr=True)),
                    ("block64_srr_bf16_wgrad", dict(scale_block_size=64, srr=True)),
                    ("block64_srr_fp8_dgrad_bf16_wgrad", dict(scale_block_size=64, srr=True)),
                    ("block64_ef", dict(scale_block_size=64)), ("bf16", None)):
        set_block_dgrad("fp8" if "fp8_dgrad" in arm else "exact")
        set_block_wgrad("bf16" if "bf16_wgrad" in arm else "split")
        torch.manual_seed(2)
        m = nn.Sequential(nn.Linear(4096, 16384), nn.GELU(), nn.Linear(16384, 4096)).to(dev)
        if kw is not None:
            convert_to_tcfp(m, use_tensor_cores=True, **kw)
        xx = x.clone().requires_grad_(False)

        def fb():
            with torch.autocast("cuda", dtype=torch.bfloat16, enabled=kw is None):
                y = m(xx)
            y.float().square().mean().backward()

        fb()
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats(dev)
        base = torch.cuda.memory_allocated(dev)
        ms = event_time_ms(fb, 5, stream, warmup=1)
        peak = torch.cuda.max_memory_allocated(dev)
        res[f"scaleup_{arm}"] = {"fwd_bwd_ms": ms, "peak_mem_MB": peak / 1e6,
                                 "resident_MB": base / 1e6}
        del m
        torch.cuda.empty_cache()
    set_block_dgrad("exact")
    set_block_wgrad("split")
    return res


def bench_c5_memory():
    """Peak-memory breakdown of the C5 scale-up layer's forward + backward
    (``Linear(4096,16384) -> GELU -> Linear(16384,4096)``, 8192 tokens):
    the caching allocator's event history of one call is replayed, and the
    allocations live at the highest point are grouped by the code that made
    them (the innermost frame in this package or this file, else the
    innermost frame).  Per arm: peak MB, resident MB (weights, EF buffers,
    optimizer-free), and the live tensors at the peak."""
    import torch
    import torch.nn as nn

    from tcfp_amd.nn import convert_to_tcfp, set_block_dgrad, set_block_wgrad

    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(0)
    x = torch.randn(8192, 4096, generator=g).bfloat16().to(dev)
    out = {}
    for arm, kw, dg, wg in (
            ("block64_srr", dict(scale_block_size=64, srr=True), "exact", "split"),
            ("block64_srr_fp8_dgrad_bf16_wgrad", dict(scale_block_size=64, srr=True), "fp8",
             "bf16"),
            ("bf16", None, "exact", "split")):
        set_block_dgrad(dg)
        set_block_wgrad(wg)
        torch.manual_seed(2)
        m = nn.Sequential(nn.Linear(4096, 16384), nn.GELU(), nn.Linear(16384, 4096)).to(dev)
        if kw is not None:
            convert_to_tcfp(m, use_tensor_cores=True, **kw)

        def fb():
            with torch.autocast("cuda", dtype=torch.bfloat16, enabled=kw is None):
                y = m(x)
            y.float().square().mean().backward()

        fb()
        for p in m.parameters():
            p.grad = None
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        live = {}
        for blk in torch.cuda.memory._snapshot()["segments"]:
            for b in blk["blocks"]:
                if b["state"] == "active_allocated":
                    live[b["address"]] = (b["size"], "resident")
        resident = sum(v[0] for v in live.values())
        torch.cuda.memory._record_memory_history(max_entries=200000)
        fb()
        torch.cuda.synchronize()
        snap = torch.cuda.memory._snapshot()
        torch.cuda.memory._record_memory_history(enabled=None)

        def where(frames):
            for f in frames:
                fn = f.get("filename", "")
                if "tcfp_amd" in fn or fn.endswith("bench.py"):
                    return f"{fn.split('/')[-1]}:{f.get('name')}:{f.get('line')}"
            f = frames[0] if frames else {}
            return f"{f.get('filename', '?').split('/')[-1]}:{f.get('name', '?')}"

        cur = dict(live)
        total = resident
        best, best_live = total, dict(cur)
        for ev in snap["device_traces"][dev.index or 0]:
            a = ev["action"]
            if a == "alloc":
                cur[ev["addr"]] = (ev["size"], where(ev.get("frames", [])))
                total += ev["size"]
                if total > best:
                    best, best_live = total, dict(cur)
            elif a == "free_completed" and ev["addr"] in cur:
                total -= cur.pop(ev["addr"])[0]
        groups = {}
        for size, w in best_live.values():
            groups[w] = groups.get(w, 0) + size
        top = sorted(groups.items(), key=lambda kv: -kv[1])
        out[arm] = {"peak_MB": best / 1e6, "resident_MB": resident / 1e6,
                    "at_peak_MB": {k: round(v / 1e6, 1) for k, v in top if v >= 1e6}}
        del m
        torch.cuda.empty_cache()
    set_block_dgrad("exact")
    set_block_wgrad("split")
    return out


def cpu_baseline(t, reps=5):
    """The reference's CPU path on the full C2 problem, timed on this box's
    host cores: its per-tensor forward with the non-fused tier
    (tcfp/nn/__init__.py:343-421) -- dual quantisation of W, activation
    quantisation (``to_fp8_e4m3`` op for op, tcfp/core.py:85-106), then
    ``X W_hi^T s s_hi + X W_lo^T s s_lo`` as fp32 matmuls of the dequantised
    operands (the product its ``torch._scaled_mm`` calls define; torch's own
    CPU ``_scaled_mm`` on FP8 takes ~15 minutes per 4096^3 product here, so
    the dequantised form stands in).  One warm-up, then the median of
    ``reps`` runs, at the thread count the box grants this process."""
    import torch

    from oracle import torch_ref as tr

    xb, w = (x.detach().cpu() for x in t[6:8])
    threads = max(1, min(os.cpu_count() or 1,
                         int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))))
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    e4m3 = torch.float8_e4m3fn

    def step():
        t0 = time.perf_counter()
        hi, ih = tr.to_fp8(w, 448.0, e4m3)
        lo, il = tr.to_fp8(w - hi.float() * ih, 448.0, e4m3)
        a, sa = tr.to_fp8(xb, 448.0, e4m3)
        t1 = time.perf_counter()
        A = a.float() * sa
        out = A @ (hi.float() * ih).t() + A @ (lo.float() * il).t()
        t2 = time.perf_counter()
        return t2 - t0, t2 - t1, out

    try:
        step()
        runs = [step()[:2] for _ in range(reps)]
    finally:
        torch.set_num_threads(prev)
    total = statistics.median(r[0] for r in runs)
    gemm = statistics.median(r[1] for r in runs)
    flop = 2 * 2 * xb.shape[0] * w.shape[0] * w.shape[1]
    return {
        "value": flop / total / 1e12, "unit": "TFLOP/s", "cores": int(threads), "kind": "port",
        "sample": (f"full configs[1] problem (4096^3): the reference's per-tensor forward on CPU "
                   f"(oracle/torch_ref.to_fp8 dual quant of W + act quant, then fp32 matmuls "
                   f"of the dequantised operands), torch {torch.__version__}, {threads} "
                   f"threads, 1 warm-up + median of {reps}: {total * 1e3:.0f} ms per step "
                   f"({gemm * 1e3:.0f} ms of it the two matmuls)"),
        "ms_per_step": total * 1e3,
        "gemm_only_tflops": flop / gemm / 1e12,
    }


def traffic_from_profiles():
    p = ROOT / "profiles" / "dual_gemm_4096_traffic.json"
    if p.exists():
        try:
            return json.loads(p.read_text()).get("hbm_bytes_per_launch")
        except Exception:
            return None
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--part", choices=("all", "gemm", "quant", "quantcold", "quantfuse", "sweep",
                                       "block", "mlp", "c5", "c5mem", "copy", "scaled_mm"),
                    default="all",
                    help="all (default) = headline + every secondary figure; the others run "
                         "one workload (for profiling)")
    ap.add_argument("--arm", choices=("both", "tcfp", "tcfp_fused", "bf16", "fp32"),
                    default="both", help="--part mlp: which model(s) to run (both = all)")
    ap.add_argument("--skip-extras", action="store_true", help="same as --part gemm")
    args = ap.parse_args()
    if args.skip_extras:
        args.part = "gemm"
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the TCFP-12 path has no "
              "multi-GPU component); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.part != "all" and args.part != "gemm":
        fn = {"quant": lambda: bench_dual_quant(), "block": lambda: bench_block_gemms(iters=20, heat=3, rounds=1),
              "c5": lambda: bench_c5(), "c5mem": lambda: bench_c5_memory(),
              "quantcold": lambda: bench_dual_quant_cold(max(1, args.steps // 20)),
              "quantfuse": lambda: bench_quant_in_consumer(),
              "sweep": lambda: bench_gemm_sweep(),
              "mlp": lambda: bench_mlp(
                  steps=args.steps,
                  arms=("tcfp", "tcfp_fused", "bf16", "fp32") if args.arm == "both"
                  else (args.arm,), rounds=5 if args.arm == "both" else 1),
              "copy": lambda: bench_copy(args.steps),
              "scaled_mm": lambda: bench_scaled_mm(args.steps, args.warmup)}
        log(f"[bench] part {args.part}")
        print(json.dumps({"part": args.part, **fn[args.part]()}), flush=True)
        return
    extras = {}
    cpu = None
    t = c2_tensors()
    if args.part == "all":
        # The secondary parts run first: they bring the GPU out of idle
        # (clock ramp-up takes longer than a few warm-up launches), so the
        # headline's timed steps see the clocks of a working GPU.
        log("[bench] CPU baseline")
        cpu = cpu_baseline(t)
        log("[bench] comparators")
        extras["comparators_4096"] = bench_comparators(t)
        log("[bench] block-scaled GEMMs (configs[2])")
        extras["block_scaled_4096"] = bench_block_gemms()
        log("[bench] dual quant")
        extras["quant_kernels"] = bench_dual_quant()
        log("[bench] MLP train step (configs[3])")
        extras["mlp_train_step"] = bench_mlp()
        log("[bench] TinyGPT + scale-up layer (configs[4])")
        extras["c5"] = bench_c5()
    log(f"[bench] dual GEMM 4096^3: warmup {args.warmup}, steps {args.steps}")
    r = bench_dual_gemm(args.steps, args.warmup, t, sustained=4000)
    log(f"[bench] dual GEMM: {r['tflops_wall']:.1f} TFLOP/s wall, {r['tflops_kern']:.1f} "
        f"TFLOP/s events, rel_fro {r['rel_fro']:.2e}")
    if "sustained_tflops" in r:
        extras["sustained_back_to_back"] = {"launches": r["sustained_launches"],
                                            "ms": r["sustained_ms"],
                                            "tflops": r["sustained_tflops"]}
    achieved = r["tflops_kern"]
    line = {
        "metric": "dual-FP8 GEMM TFLOP/s @4096^3 (% FP8 MFMA peak); MLP train-step ms",
        "value": round(r["tflops_wall"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["wall_ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3 (fp32 accumulate, bf16 out)",
        "data": "synthetic (seeded randn, bf16 X quantised per-tensor, fp32 W dual-quantised)",
        "config": {"workload": "configs[1]: fused dual FP8 GEMM, per-tensor scales, "
                               "M=N=K=4096, bf16 out", "M": 4096, "N": 4096, "K": 4096,
                   "parallelism": "single GPU"},
        "pct_fp8_peak": round(100 * r["tflops_wall"] / FP8_PEAK_TFLOPS, 2),
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": FP8_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / FP8_PEAK_TFLOPS, 4),
                     "traffic": traffic_from_profiles()},
        "cpu_baseline": cpu,
        "parity_rel_fro": r["rel_fro"],
        **extras,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
