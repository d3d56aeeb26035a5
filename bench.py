"""Benchmark of the fused MoE on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c3_t8192]
                    [--sweep | --no-sweep] [--no-cpu] [--no-pmc]

A step is one call of ``flashinfer_amd.kernel.run`` on the workload's
synthetic inputs, already resident in HBM. The headline workload is the
prefill point T=8192 (H=7168, I=2048, 32 local experts of 256, top-8, FP8
e4m3 block-scaled; 11,559 local slots over 28 active experts), the largest
of the metric's T = 1 / 256 / 8192, where the grouped GEMMs are bound by
the matrix cores. W untimed calls, then 5 trials of K calls each, bracketed
by ``torch.cuda.synchronize()``; ``value`` is the median trial's
microseconds per call. A second pass of 5 x K calls records HIP events
between the kernels on the stream they run on, which gives each kernel's
average duration. A third pass times single calls with the caches cold (a
512 MiB read before each call evicts the MALL and L2s), a fourth replays the
call captured in a HIP graph, and the probes of libmi_peaks.so measure the
HBM and MFMA rates this GPU achieves.

Rank 0 prints ONE JSON line. ``roofline`` covers the dominant kernel
(GEMM1+SwiGLU; at T=8192 bound by FP8 MFMA), with HBM traffic and the MFMA
busy fraction from rocprofv3 counter passes; ``kernels`` gives both GEMMs'
rooflines; ``call_roofline`` the whole call; ``sweep`` every configuration
(the headline included), each with its dominant kernel's roofline, a
``parity`` block and, at the CPU reference configuration (T=16) and the
metric's points (T = 1 with and without a local slot, 256, 8192), the CPU
oracle timed on this host (``cpu_baseline``); ``quantize_fp8`` the
activation quantiser that feeds the operator.

``parity`` mirrors the per-workload correctness fields the reference
harness prints beside its latency (scripts/run_local.py:65-78): after all
GPU timing, the CPU oracle runs on the same seeded inputs (every token up to
T = 1024, 256 tokens spread over [0, T) above) and the GPU output of the
timed calls is compared with its fp32 accumulator: routing top-k set
mismatches (must be 0) and tokens with a selection boundary within 4 fp32
ulps, max absolute error, max relative error over the elements with
|ref| >= 1 % of max|ref|, normwise error, and the fraction of elements
outside |out - ref| <= 1e-2 |ref| + 1e-2 max|ref|.
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import shutil
import statistics
import subprocess
import sys
import tempfile
import time

import torch

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, GB/s
FP8_PEAK_TFLOPS = 5000.0     # dense FP8 MFMA, TFLOP/s
BF16_PEAK_TFLOPS = 2500.0    # dense BF16 MFMA, TFLOP/s
H, I, E_GLOBAL, BLOCK = 7168, 2048, 256, 128

# Algorithmic bytes: weights + block scales of each active expert, plus the
# per-token and per-slot rows a kernel must read or write once.
W1_EXPERT_BYTES = 2 * I * H + (2 * I // BLOCK) * (H // BLOCK) * 4        # 29,367,296
W2_EXPERT_BYTES = H * I + (H // BLOCK) * (I // BLOCK) * 4                # 14,683,648
HS_ROW_BYTES = H + (H // BLOCK) * 4                                      # fp8 row + scales
ACT_ROW_BYTES = I * 2                                                    # bf16 SwiGLU row
PART_ROW_BYTES = H * 2                                                   # bf16 weighted GEMM2 row
GEMM1_FLOPS_PER_SLOT = 2 * 2 * I * H
GEMM2_FLOPS_PER_SLOT = 2 * H * I

HEADLINE = "c3_t8192"
SWEEP = ["c0_t16", "c1_t1", "c1_t1_local", "c1_t4", "c1_t16", "c1_t64", "t256", "c2_t1024_o0",
         "c3_t8192", "c4_t14000_skew"]
# The CPU reference configuration (T = 16) and the metric's points (T = 1 /
# 256 / 8192): each sweep entry of these carries the CPU oracle timed on this
# host beside the GPU figures.
CPU_POINTS = ("c0_t16", "c1_t1", "c1_t1_local", "t256", "c3_t8192")
PARITY_ALL_T = 1024   # parity on every token up to this T, on a spread subset above
PARITY_SUBSET = 256


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def call_bytes(T, A_e):
    return T * (E_GLOBAL * 4 + HS_ROW_BYTES + H * 2) + E_GLOBAL * 2 + A_e * (W1_EXPERT_BYTES + W2_EXPERT_BYTES)


def gemm1_bytes(S, A_e):
    return A_e * W1_EXPERT_BYTES + S * (HS_ROW_BYTES + ACT_ROW_BYTES)


def gemm2_bytes(S, A_e):
    return A_e * W2_EXPERT_BYTES + S * (ACT_ROW_BYTES + PART_ROW_BYTES)


def kernel_rooflines(res):
    """Roofline of each GEMM launch from its average duration (HIP events):
    the binding bound is the larger of its algorithmic HBM bytes at 8 TB/s
    and its flops at the matrix-core peak of the type it computes in (GEMM1
    FP8, GEMM2 bf16); ``frac`` = that bound time / measured time."""
    S, A_e = res["slots"], res["active_experts"]
    out = {}
    for name, nbytes, flops, peak, dtype in (
            ("gemm1_swiglu", gemm1_bytes(S, A_e), S * GEMM1_FLOPS_PER_SLOT, FP8_PEAK_TFLOPS, "fp8"),
            ("gemm2", gemm2_bytes(S, A_e), S * GEMM2_FLOPS_PER_SLOT, BF16_PEAK_TFLOPS, "bf16")):
        us = res["phase_us"][name]
        if S == 0 or us <= 0:
            out[name] = {"bound": "latency", "note": "no local slot: nothing to stream or multiply",
                         "avg_launch_us": us}
            continue
        t = us * 1e-6
        t_hbm = nbytes / (HBM_PEAK_GBS * 1e9)
        t_mfma = flops / (peak * 1e12)
        if t_mfma >= t_hbm:
            r = {"bound": "mfma", "achieved": round(flops / t / 1e12, 1), "peak": peak,
                 "unit": "TFLOP/s", "mfma_dtype": dtype}
        else:
            r = {"bound": "hbm", "achieved": round(nbytes / t / 1e9, 1), "peak": HBM_PEAK_GBS,
                 "unit": "GB/s"}
        r["frac"] = round(max(t_hbm, t_mfma) / t, 4)
        r.update({"avg_launch_us": round(us, 2), "algorithmic_bytes_per_launch": nbytes,
                  "algorithmic_flops_per_launch": flops,
                  "gbps": round(nbytes / t / 1e9, 1), "tflops": round(flops / t / 1e12, 1)})
        out[name] = r
    return out


def make(name):
    from flashinfer_amd import workloads as W
    return W.standard(name)


def routing_stats(T):
    from flashinfer_amd import _lib, kernel
    L = _lib.workspace_layout(T)
    eoff = kernel.last_workspace()[L.expert_off:L.expert_off + 33 * 4].view(torch.int32).cpu()
    counts = (eoff[1:] - eoff[:-1]).tolist()
    return int(eoff[-1]), sum(1 for c in counts if c > 0), max(counts) if counts else 0


_DEV_W = {}


def device_args(wl, dev):
    """Per-token tensors copied to the GPU; the shared weights are copied once."""
    names = ["gemm1_weights", "gemm1_weights_scale", "gemm2_weights", "gemm2_weights_scale"]
    if not _DEV_W:
        for n in names:
            _DEV_W[n] = wl.tensors[n].to(dev)
    t = wl.tensors
    return [t["routing_logits"].to(dev), t["routing_bias"].to(dev), t["hidden_states"].to(dev),
            t["hidden_states_scale"].to(dev)] + [_DEV_W[n] for n in names] + [
        wl.local_expert_offset, wl.routed_scaling_factor]


WARM_S = 0.05         # untimed calls after the warmup count, so clocks have ramped up
MIN_TRIAL_US = 4000.0  # sweep entries: calls per trial raised to fill at least this


def time_workload(wl, steps, warmup, trials=5, exact=True):
    """Times ``steps`` calls per trial (exact=True, the headline), or for a
    sweep entry enough calls that a trial lasts MIN_TRIAL_US, after
    ``warmup`` calls and then WARM_S of untimed calls (a 20-call trial of a
    40 us call would otherwise run partly at the clocks of the idle GPU
    that preceded it: ~10 % slower at T = 4 and 16)."""
    from flashinfer_amd import _lib, kernel
    dev = torch.device("cuda", 0)
    args = device_args(wl, dev)
    out = torch.empty(wl.T, H, dtype=torch.bfloat16, device=dev)
    for _ in range(warmup):
        kernel.run(*args, out)
    torch.cuda.synchronize()
    n_warm, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < WARM_S:
        for _ in range(10):
            kernel.run(*args, out)
        torch.cuda.synchronize()
        n_warm += 10
    est_us = (time.perf_counter() - t0) * 1e6 / n_warm
    calls = steps if exact else max(steps, int(MIN_TRIAL_US / est_us) + 1)
    S, A_e, max_rows = routing_stats(wl.T)
    # value: plain calls, trials x calls, bracketed by synchronize
    trial_us = []
    for tr in range(trials):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for k in range(calls):
            kernel.run(*args, out)
        torch.cuda.synchronize()
        trial_us.append((time.perf_counter() - t0) * 1e6 / calls)
    # per-kernel durations: the same calls with HIP events recorded between the
    # kernels on their stream (the records add a little time between kernels)
    nev = _lib.NUM_PHASES + 1
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(nev)] for _ in range(steps)]
    phase_sum = [0.0] * _lib.NUM_PHASES
    prof_us = []
    for tr in range(trials):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for k in range(steps):
            kernel.run_profiled(*args, out, events=ev[k])
        torch.cuda.synchronize()
        prof_us.append((time.perf_counter() - t0) * 1e6 / steps)
        for k in range(steps):
            for p in range(_lib.NUM_PHASES):
                phase_sum[p] += ev[k][p].elapsed_time(ev[k][p + 1]) * 1e3
    phase_us = [s / (steps * trials) for s in phase_sum]
    cold_us = time_cold(args, out, min(steps, 20))
    graph_us = time_graph(args, out, calls)
    us = statistics.median(trial_us)
    B = call_bytes(wl.T, A_e)
    F1, F2 = S * GEMM1_FLOPS_PER_SLOT, S * GEMM2_FLOPS_PER_SLOT
    F = F1 + F2
    t = us * 1e-6
    bound_t = max(B / (HBM_PEAK_GBS * 1e9), F / (FP8_PEAK_TFLOPS * 1e12))
    # GEMM2 runs on bf16 MFMA: the bound with its flops priced at the bf16 peak
    mixed_t = max(B / (HBM_PEAK_GBS * 1e9),
                  F1 / (FP8_PEAK_TFLOPS * 1e12) + F2 / (BF16_PEAK_TFLOPS * 1e12))
    res = {
        "workload": wl.name, "T": wl.T, "local_expert_offset": wl.local_expert_offset,
        "slots": S, "active_experts": A_e, "max_rows_per_expert": max_rows,
        "us_per_call": round(us, 2), "trials_us": [round(x, 2) for x in trial_us],
        "calls_per_trial": calls,
        "us_per_call_with_phase_events": round(statistics.median(prof_us), 2),
        "gbps": round(B / t / 1e9, 1), "tflops": round(F / t / 1e12, 2),
        "hbm_frac": round(B / t / 1e9 / HBM_PEAK_GBS, 4),
        "fp8_frac": round(F / t / 1e12 / FP8_PEAK_TFLOPS, 4),
        "roofline_frac": round(bound_t / t, 4),
        "mixed_roofline_frac": round(mixed_t / t, 4),
        "us_per_call_cold": round(cold_us, 2),
        "us_per_call_graph": round(graph_us, 2),
        "algorithmic_bytes": B, "algorithmic_flops": F,
        "phase_us": {n: round(v, 2) for n, v in zip(_lib.PHASES, phase_us)},
    }
    g1 = phase_us[2] * 1e-6
    g2 = phase_us[3] * 1e-6
    res["gemm1_gbps"] = round(gemm1_bytes(S, A_e) / g1 / 1e9, 1) if g1 > 0 else None
    res["gemm1_tflops"] = round(F1 / g1 / 1e12, 2) if g1 > 0 else None
    res["gemm2_gbps"] = round(gemm2_bytes(S, A_e) / g2 / 1e9, 1) if g2 > 0 else None
    res["gemm2_tflops"] = round(F2 / g2 / 1e12, 2) if g2 > 0 else None
    res["kernels"] = kernel_rooflines(res)
    # the dominant kernel: the GEMM launch that takes longest
    dom = max(res["kernels"], key=lambda k: res["phase_us"][k])
    res["roofline"] = dict(res["kernels"][dom], kernel=dom)
    # the timed calls' output rows and routing for the parity check in the
    # CPU leg (the call is deterministic: every call wrote the same bytes)
    tok = parity_tokens(wl.T)
    ids, _ = kernel.route(args[0], args[1], wl.routed_scaling_factor)
    res["_check"] = {"tokens": tok, "out": out[tok.to(dev)].cpu(), "ids": ids[tok.to(dev)].cpu()}
    del args, out
    return res


def parity_tokens(T):
    """Every token up to PARITY_ALL_T, else PARITY_SUBSET spread over [0, T)
    with the first and the last."""
    if T <= PARITY_ALL_T:
        return torch.arange(T)
    return torch.unique(torch.linspace(0, T - 1, PARITY_SUBSET).round().long())


def parity_block(wl, chk):
    """The CPU oracle on the checked tokens of ``wl`` (tokens are independent,
    so every per-token input is sliced) against the GPU rows of the timed
    calls; see the module docstring for the fields."""
    from oracle import ref_moe as R
    tok = chk["tokens"]
    t = wl.tensors
    ng, kg, k = wl.routing
    sub = [t["routing_logits"][tok], t["routing_bias"], t["hidden_states"][tok],
           t["hidden_states_scale"][:, tok].contiguous(), t["gemm1_weights"],
           t["gemm1_weights_scale"], t["gemm2_weights"], t["gemm2_weights_scale"],
           wl.local_expert_offset, wl.routed_scaling_factor]
    ref = R.moe_forward(*sub, n_group=ng, topk_group=kg, top_k=k)
    rep = R.tolerance_report(chk["out"].float(), ref.acc)
    o, r = chk["out"].double(), ref.acc.double()
    big = r.abs() >= 0.01 * float(r.abs().max()) if r.numel() else r.bool()
    max_rel = float(((o - r).abs()[big] / r.abs()[big]).max()) if big.any() else 0.0
    mism = R.routing_set_mismatch(chk["ids"], ref.route.ids)
    ties = R.near_tie_tokens(sub[0], sub[1], ng, kg, k)
    return {"tokens_checked": int(tok.numel()), "of_tokens": wl.T,
            "routing_set_mismatches": int(mism), "near_tie_tokens": int(ties),
            "max_abs_err": float(f"{rep['max_abs_err']:.3e}"), "max_rel_err": float(f"{max_rel:.3e}"),
            "normwise_rel": float(f"{rep['normwise_rel']:.3e}"),
            "frac_outside": float(f"{rep['frac_bad']:.3e}"),
            "pass": bool(mism == 0 and rep["n_bad"] == 0)}


def compact(res):
    """A sweep entry of the JSON line: the figures a reader compares across
    configurations (the headline's full record stays at the top level)."""
    keep = ("workload", "T", "slots", "active_experts", "us_per_call", "us_per_call_cold",
            "us_per_call_graph", "gbps", "tflops", "roofline_frac", "mixed_roofline_frac")
    out = {k: res[k] for k in keep}
    out["phase_us"] = {k: round(v, 1) for k, v in res["phase_us"].items()}
    rf = res["roofline"]
    out["roofline"] = {k: rf[k] for k in ("kernel", "bound", "achieved", "unit", "frac", "avg_launch_us")
                       if k in rf}
    for k in ("parity", "cpu_baseline"):
        if k in res:
            out[k] = res[k]
    return out


def time_graph(args, out, steps, trials=5):
    """Median microseconds per call when the call is captured once in a HIP
    graph and replayed (launch overheads of the five kernels shrink)."""
    from flashinfer_amd import kernel
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        kernel.run(*args, out)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        kernel.run(*args, out)
    g.replay()
    torch.cuda.synchronize()
    ts = []
    for _ in range(trials):
        t0 = time.perf_counter()
        for _ in range(steps):
            g.replay()
        torch.cuda.synchronize()
        ts.append((time.perf_counter() - t0) * 1e6 / steps)
    del g
    return statistics.median(ts)


def time_cold(args, out, steps, flush_mib=512):
    """Median microseconds of one call with the caches cold: before each call
    a 512 MiB read evicts the 256 MB MALL and the L2s (a read, so no dirty
    lines are written back during the call); HIP events on the call's stream
    bracket the call alone."""
    from flashinfer_amd import kernel
    flush = torch.ones((flush_mib << 20) // 4, dtype=torch.float32, device=out.device)
    sink = torch.empty((), dtype=torch.float32, device=out.device)
    ts = []
    for _ in range(steps):
        torch.sum(flush, dim=0, out=sink)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        kernel.run(*args, out)
        e1.record()
        e1.synchronize()
        ts.append(e0.elapsed_time(e1) * 1e3)
    del flush
    return statistics.median(ts)


def time_quantizer(T, reps=50):
    """The FP8 activation quantiser on bf16 [T, 7168]: median µs per call and
    HBM rate (2 B read + 1 B written per element, plus the [56, T] scales)."""
    from flashinfer_amd import kernel
    g = torch.Generator(device="cuda").manual_seed(T)
    x = torch.randn(T, H, device="cuda", generator=g).to(torch.bfloat16)
    q = torch.empty(T, H, dtype=torch.float8_e4m3fn, device="cuda")
    s = torch.empty(H // BLOCK, T, dtype=torch.float32, device="cuda")
    kernel.quantize_activations(x, q, s)
    ts = []
    for _ in range(5):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            kernel.quantize_activations(x, q, s)
        e1.record()
        e1.synchronize()
        ts.append(e0.elapsed_time(e1) * 1e3 / reps)
    us = statistics.median(ts)
    nbytes = T * H * 3 + T * (H // BLOCK) * 4
    return {"T": T, "us_per_call": round(us, 2), "bytes": nbytes,
            "gbps": round(nbytes / (us * 1e-6) / 1e9, 1),
            "hbm_frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}


def vendor_gemm_reference():
    """Plain GEMMs of the operator's shapes through the vendor library
    (torch._scaled_mm -> hipBLASLt for fp8, torch.matmul for bf16): per-tensor
    scales, contiguous operands, no gather, no block scales, no SwiGLU. A
    yardstick for the fused grouped kernels, not part of the operator."""
    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(0)
    rows = []

    def timed(fn, reps=20):
        fn()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        e1.synchronize()
        return e0.elapsed_time(e1) * 1e3 / reps

    one = torch.tensor(1.0, device=dev)
    for M in (256, 416, 1024, 4096, 14000):  # GEMM1: [M, 7168] x [4096, 7168]^T, fp8
        a = torch.randn(M, H, device=dev, generator=g).to(torch.float8_e4m3fn)
        b = torch.randn(2 * I, H, device=dev, generator=g).to(torch.float8_e4m3fn)
        us = timed(lambda: torch._scaled_mm(a, b.t(), scale_a=one, scale_b=one,
                                            out_dtype=torch.bfloat16))
        rows.append({"gemm": "fp8 M x 4096 x 7168", "M": M, "us": round(us, 1),
                     "tflops": round(2 * M * 2 * I * H / us / 1e6, 1)})
    for M in (416, 4096, 14000):  # GEMM2: [M, 2048] x [7168, 2048]^T, bf16
        a = torch.randn(M, I, device=dev, generator=g, dtype=torch.bfloat16)
        b = torch.randn(H, I, device=dev, generator=g, dtype=torch.bfloat16)
        us = timed(lambda: a @ b.t())
        rows.append({"gemm": "bf16 M x 7168 x 2048", "M": M, "us": round(us, 1),
                     "tflops": round(2 * M * H * I / us / 1e6, 1)})
    return rows


def measured_peaks():
    """Achievable rates on this GPU, from the probes in libmi_peaks.so
    (include/mi_peaks.h): an HBM read and copy (best workgroup count of a
    small sweep, median of 5 launches each) and dense fp8 / bf16 MFMA loops."""
    import ctypes
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "flashinfer_amd",
                        "libmi_peaks.so")
    if not os.path.exists(path):
        log("[bench] libmi_peaks.so missing; measured peaks skipped")
        return None
    L = ctypes.CDLL(path)
    vp, i32, i64, sz = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_size_t
    L.mi_peak_read.argtypes = [vp, sz, i32, vp, vp]
    L.mi_peak_copy.argtypes = [vp, vp, sz, i32, vp]
    L.mi_peak_mfma.argtypes = [i32, i64, i32, vp, vp]
    L.mi_peak_mfma_flops.argtypes = [i32, i64, i32]
    L.mi_peak_mfma_flops.restype = ctypes.c_double
    stream = vp(torch.cuda.current_stream().cuda_stream)

    def best(launch, reps=5):
        launch()
        ts = []
        for _ in range(reps):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            rc = launch()
            e1.record()
            e1.synchronize()
            if rc != 0:
                raise RuntimeError(f"peak probe returned {rc}")
            ts.append(e0.elapsed_time(e1) * 1e-3)
        return statistics.median(ts)

    nbytes = 2 << 30
    a = torch.ones(nbytes, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    sink = torch.zeros(8192 * 256, dtype=torch.float32, device="cuda")
    wgs = (512, 1024, 2048, 4096)
    read = max(nbytes / best(lambda: L.mi_peak_read(a.data_ptr(), nbytes, wg, sink.data_ptr(), stream))
               for wg in wgs)
    half = nbytes // 2
    copy = max(2 * half / best(lambda: L.mi_peak_copy(b.data_ptr(), a.data_ptr(), half, wg, stream))
               for wg in wgs)
    del a, b
    out = {"hbm_read_gbs": round(read / 1e9, 1), "hbm_copy_gbs": round(copy / 1e9, 1),
           "copy_counts": "read + write bytes"}
    for kind, key in ((0, "fp8_mfma_tflops"), (1, "bf16_mfma_tflops")):
        rates = []
        for wg in (512, 1024):
            iters = 4000 if kind == 0 else 8000
            t = best(lambda: L.mi_peak_mfma(kind, iters, wg, sink.data_ptr(), stream), reps=3)
            rates.append(L.mi_peak_mfma_flops(kind, iters, wg) / t)
        out[key] = round(max(rates) / 1e12, 1)
    del sink
    return out


def profiler_inherited(env=None) -> bool:
    """True when this process runs under a profiler: rocprofv3 preloads its
    tool library (LD_PRELOAD, ROCP_TOOL_LIBRARIES), which initialises the GPU
    before the program starts, so no child may be started from here."""
    env = os.environ if env is None else env
    if env.get("ROCP_TOOL_LIBRARIES") or env.get("HSA_TOOLS_LIB"):
        return True
    preload = env.get("LD_PRELOAD", "")
    return any(k in preload for k in ("rocprof", "roctracer", "rocprofiler"))


def _pmc_pass(counters, workload, copy_mib, timeout):
    """One rocprofv3 counter pass over a short child run of this bench on
    ``workload`` (which also copies ``copy_mib`` MiB device-to-device first).
    Returns {counter: {kernel name: [per-dispatch values]}}, or None."""
    exe = shutil.which("rocprofv3")
    if exe is None:
        return None
    env = dict(os.environ, TMPDIR="/tmp")
    with tempfile.TemporaryDirectory(dir="/tmp") as d:
        cmd = ["timeout", "-s", "KILL", str(timeout), exe, "--pmc", *counters, "--output-format",
               "csv", "-d", d, "-o", "pmc", "--", sys.executable, "-u",
               os.path.abspath(__file__), "--workload", workload, "--steps", "2",
               "--warmup", "1", "--no-sweep", "--no-cpu", "--no-pmc",
               "--copy-calib-mib", str(copy_mib)]
        log(f"[bench] counter pass {' '.join(counters)} ...")
        r = subprocess.run(cmd, capture_output=True, text=True, env=env, cwd="/tmp")
        files = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
        if r.returncode != 0 or not files:
            log(f"[bench] counter pass {' '.join(counters)} failed (rc={r.returncode})")
            return None
        vals = {c: {} for c in counters}
        with open(files[0]) as f:
            for row in csv.DictReader(f):
                c = row["Counter_Name"]
                if c in vals:
                    vals[c].setdefault(row["Kernel_Name"], []).append(float(row["Counter_Value"]))
        return vals


def _pick(per_kernel, key):
    """Median per-dispatch value over the kernels whose name contains key."""
    xs = [v for name, vs in per_kernel.items() if key in name for v in vs]
    return statistics.median(xs) if xs else None


def pmc_counters(workload, kernel_key, copy_mib=1024, timeout=240):
    """Counters of the first kernel whose name contains ``kernel_key``, from
    three rocprofv3 passes over short child runs of this bench (each pass a
    process of its own): HBM bytes per launch from FETCH_SIZE and WRITE_SIZE,
    each scaled to bytes by what the same counter reads for a device copy of
    ``copy_mib`` MiB timed in the same pass; and the MFMA busy fraction,
    SQ_VALU_MFMA_BUSY_CYCLES per SIMD (1024 SIMDs) over GRBM_GUI_ACTIVE per
    XCD (8 XCDs). Returns None, starting nothing, if rocprofv3 is
    unavailable or this process itself runs under a profiler; fields of a
    failed pass are null. Must run before this process touches the GPU."""
    if profiler_inherited():
        log("[bench] running under a profiler: counter passes skipped (traffic = null)")
        return None
    if shutil.which("rocprofv3") is None:
        return None
    out = {"kernel_key": kernel_key, "copy_bytes": copy_mib << 20}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        vals = _pmc_pass([counter], workload, copy_mib, timeout)
        key = "fetch" if counter == "FETCH_SIZE" else "write"
        k_units = _pick(vals[counter], kernel_key) if vals else None
        c_units = max((v for name, vs in vals[counter].items() if "copyBuffer" in name
                       for v in vs), default=None) if vals else None
        if k_units is None or not c_units:
            out[f"{key}_bytes"] = None
            continue
        scale = (copy_mib << 20) / c_units
        out[f"{key}_counter"] = k_units
        out[f"{key}_copy_counter"] = c_units
        out[f"{key}_scale"] = round(scale, 4)
        out[f"{key}_bytes"] = k_units * scale
    fb, wb = out.get("fetch_bytes"), out.get("write_bytes")
    out["bytes"] = fb + wb if fb is not None and wb is not None else None
    vals = _pmc_pass(["SQ_VALU_MFMA_BUSY_CYCLES", "GRBM_GUI_ACTIVE"], workload, 0, timeout)
    busy = _pick(vals["SQ_VALU_MFMA_BUSY_CYCLES"], kernel_key) if vals else None
    gui = _pick(vals["GRBM_GUI_ACTIVE"], kernel_key) if vals else None
    out["mfma_busy_cycles"] = busy
    out["gui_active_cycles"] = gui
    out["mfma_busy_frac"] = round((busy / 1024) / (gui / 8), 4) if busy and gui else None
    return out


def host_cores():
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_baseline(wl, reps):
    """The CPU oracle (fp32 torch) on this host's cores: 1 warmup + ``reps``
    timed calls of the whole workload (the oracle dequantises only the active
    experts' weights), median."""
    from oracle import ref_moe as R
    torch.set_num_threads(host_cores())
    cores = torch.get_num_threads()
    args = wl.args()
    R.moe_forward(*args)
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        R.moe_forward(*args)
        ts.append(time.perf_counter() - t0)
    return {"value": round(statistics.median(ts) * 1e6, 1), "unit": "us/call", "cores": cores,
            "kind": "port",
            "sample": f"full {wl.name} call (T={wl.T}), fp32 torch oracle dequantising only the "
                      f"active experts, 1 warmup + {reps} timed, median"}


def full_dequant_call_us(wl):
    """One whole call of the CPU oracle in the definition-style schedule that
    dequantises all 32 local experts' weights on every call (one timed call
    after the active-experts warmup)."""
    from oracle import ref_moe as R
    t0 = time.perf_counter()
    R.moe_forward(*wl.args(), dequant_all_experts=True)
    return round((time.perf_counter() - t0) * 1e6, 1)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default=HEADLINE)
    ap.add_argument("--sweep", dest="sweep", action="store_true", default=True)
    ap.add_argument("--no-sweep", dest="sweep", action="store_false")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-pmc", action="store_true",
                    help="skip the rocprofv3 counter passes (traffic and MFMA busy = null)")
    ap.add_argument("--vendor-gemm-ref", action="store_true",
                    help="only time plain vendor-library GEMMs of the operator's shapes and "
                         "print them as one JSON line")
    ap.add_argument("--copy-calib-mib", type=int, default=0,
                    help="(counter passes) copy this many MiB device-to-device before timing")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this operator is one expert-parallel shard "
              "(local_expert_offset selects the shard) and has no multi-GPU path. "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    counters = None
    if not a.no_pmc and not a.vendor_gemm_ref:
        # counter passes run as child processes before this one uses the GPU;
        # the dominant kernel at the headline is the LDS-tiled GEMM1 above
        # T = 1536, the K-split or wide GEMM1 below
        from flashinfer_amd import workloads as W
        key = "gemm1_tile" if W.STANDARD[a.workload]["T"] > 1536 else "gemm1_"
        counters = pmc_counters(a.workload, key)
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(2)
    if a.vendor_gemm_ref:
        print(json.dumps({"vendor_gemm_reference": vendor_gemm_reference()}), flush=True)
        return
    if a.copy_calib_mib > 0:
        src = torch.empty(a.copy_calib_mib << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    from flashinfer_amd import _lib
    _lib.lib()

    t_start = time.time()
    wl = make(a.workload)
    log(f"[bench] inputs for {a.workload} ready in {time.time() - t_start:.1f}s")
    head = time_workload(wl, a.steps, a.warmup)

    def loggable(r):
        return {k: v for k, v in r.items() if not k.startswith("_")}

    log(f"[bench] {json.dumps(loggable(head))}")
    sweep = []
    if a.sweep:
        for name in SWEEP:
            if name == a.workload:
                sweep.append(head)
                continue
            w = make(name)
            steps = a.steps if w.T <= 1024 else max(10, a.steps // 2)
            r = time_workload(w, steps, a.warmup, exact=False)
            log(f"[bench] {json.dumps(loggable(r))}")
            sweep.append(r)
            del w
    else:
        sweep.append(head)
    quant = [time_quantizer(T) for T in (64, 8192)] if a.sweep else []
    for qr in quant:
        log(f"[bench] quantiser {qr}")
    peaks = None
    if a.copy_calib_mib == 0:  # not in the counter passes: their largest copy calibrates
        peaks = measured_peaks()
        log(f"[bench] measured peaks {peaks}")

    cpu = None
    if not a.no_cpu:
        # The CPU leg, after all GPU timing: the oracle checks every entry's
        # GPU output (parity), and is timed at the CPU reference
        # configuration and the metric's points (1 timed call above T = 1024,
        # 3 below); at the headline also in the full-dequant schedule.
        for r in sweep:
            w = make(r["workload"])
            r["parity"] = parity_block(w, r.pop("_check"))
            log(f"[bench] parity {w.name} {r['parity']}")
            if r["workload"] in CPU_POINTS or r is head:
                log(f"[bench] CPU oracle baseline {w.name} ...")
                r["cpu_baseline"] = cpu_baseline(w, 1 if w.T > 1024 else 3)
                if r is head:
                    r["cpu_baseline"]["full_dequant_call_us"] = full_dequant_call_us(w)
                log(f"[bench] cpu {w.name} {r['cpu_baseline']}")
            del w
        cpu = head["cpu_baseline"]
    for r in sweep:
        r.pop("_check", None)

    roof = dict(head["roofline"])
    if counters:
        roof["traffic"] = round(counters["bytes"]) if counters.get("bytes") else None
        roof["mfma_busy_frac"] = counters.get("mfma_busy_frac")
    else:
        roof["traffic"] = None
    if peaks and roof.get("bound") == "mfma":
        meas = peaks["fp8_mfma_tflops"] if roof.get("mfma_dtype") == "fp8" else peaks["bf16_mfma_tflops"]
        roof["measured_peak"] = meas
        roof["frac_of_measured_peak"] = round(roof["achieved"] / meas, 4)
    elif peaks and roof.get("bound") == "hbm":
        roof["measured_peak"] = peaks["hbm_read_gbs"]
        roof["frac_of_measured_peak"] = round(roof["achieved"] / peaks["hbm_read_gbs"], 4)
    line = {
        "metric": "fused-MoE µs/call + FP8 TFLOP/s & HBM GB/s vs roofline at T=1/256/8192",
        "value": head["us_per_call"], "unit": "us/call", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(head["us_per_call"] / 1000.0, 5),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp8_e4m3 (GEMM1) / bf16 (GEMM2), fp32 accumulate",
        "data": "synthetic (seeded N(0,1) fp8 weights/activations, U scales, N(0,0.1) bias)",
        "config": {"workload": f"{wl.name}: one fused-MoE layer call, T={wl.T} tokens", "T": wl.T,
                   "H": H, "I": I, "experts_global": E_GLOBAL, "experts_local": 32, "top_k": 8,
                   "local_expert_offset": wl.local_expert_offset,
                   "slots": head["slots"], "active_experts": head["active_experts"],
                   "parallelism": "single GPU (one EP shard)"},
        "roofline": roof,
        "kernels": head["kernels"],
        "measured_peaks": peaks,
        "call_roofline": {"gbps": head["gbps"], "hbm_frac": head["hbm_frac"],
                          "tflops": head["tflops"], "roofline_frac": head["roofline_frac"],
                          "mixed_roofline_frac": head["mixed_roofline_frac"],
                          "us_per_call_cold": head["us_per_call_cold"],
                          "us_per_call_graph": head["us_per_call_graph"],
                          "phase_us": head["phase_us"]},
        "counters": counters,
        "cpu_baseline": cpu,
        "parity": head.get("parity"),
        "sweep": [compact(r) for r in sweep],
        "quantize_fp8": quant,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
